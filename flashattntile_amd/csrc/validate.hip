// validate.hip -- the device half of the paged-cache validation: one launch
// reduces seq_lens and the used page-table entries to the five numbers the
// host checks (flashattn_tile/paging.py:84-130 validate_cache, as called by
// flashattn_tile/kernels/decode.py:503-522), instead of a dozen framework
// reductions.  The host copies the five numbers back once.
#include <limits.h>

#include "fat_common.h"

namespace fat {

constexpr int kStatsThreads = 1024;

// out[0..4] = min(seq_lens), max(seq_lens), min and max of page_table[b, c]
// over every row b and column c < min(ceil(max_len / P), max_pages) (INT_MAX
// and INT_MIN when no entry is used), sum_b ceil(max(seq_lens[b], 0) / P).
__global__ __launch_bounds__(kStatsThreads) void cache_stats_kernel(const int32_t* __restrict__ lens,
                                                                    const int32_t* __restrict__ pt, int B,
                                                                    int max_pages, int64_t pt_sb, int P,
                                                                    int64_t* __restrict__ out) {
  __shared__ int s_min[kStatsThreads / 64], s_max[kStatsThreads / 64];
  __shared__ long long s_sum[kStatsThreads / 64];
  __shared__ int s_need;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  int mn = INT_MAX, mx = INT_MIN;
  long long pages = 0;
  for (int b = tid; b < B; b += kStatsThreads) {
    const int l = lens[b];
    mn = min(mn, l);
    mx = max(mx, l);
    pages += (max(l, 0) + (long long)P - 1) / P;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mn = min(mn, __shfl_xor(mn, off));
    mx = max(mx, __shfl_xor(mx, off));
    pages += __shfl_xor(pages, off);
  }
  if (lane == 0) {
    s_min[w] = mn;
    s_max[w] = mx;
    s_sum[w] = pages;
  }
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < kStatsThreads / 64; ++i) {
      mn = min(mn, s_min[i]);
      mx = max(mx, s_max[i]);
      pages += s_sum[i];
    }
    out[0] = mn;
    out[1] = mx;
    out[4] = pages;
    // Columns the longest sequence uses (as the torch restatement: floor((max + P - 1) / P)).
    const long long need = mx > 0 ? ((long long)mx + P - 1) / P : 0;
    s_need = (int)min(need, (long long)max_pages);
  }
  __syncthreads();
  const int need = s_need;
  int pmn = INT_MAX, pmx = INT_MIN;
  const long long n = (long long)B * need;
  for (long long i = tid; i < n; i += kStatsThreads) {
    const int b = (int)(i / need);
    const int c = (int)(i - (long long)b * need);
    const int v = pt[b * pt_sb + c];
    pmn = min(pmn, v);
    pmx = max(pmx, v);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    pmn = min(pmn, __shfl_xor(pmn, off));
    pmx = max(pmx, __shfl_xor(pmx, off));
  }
  __syncthreads();  // s_min / s_max are reused
  if (lane == 0) {
    s_min[w] = pmn;
    s_max[w] = pmx;
  }
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < kStatsThreads / 64; ++i) {
      pmn = min(pmn, s_min[i]);
      pmx = max(pmx, s_max[i]);
    }
    out[2] = pmn;
    out[3] = pmx;
  }
}

}  // namespace fat

extern "C" int fat_cache_stats(const fat_cache_stats_args* a, void* stream_ptr) {
  fat_host::clear_error();
  if (!a || !a->seq_lens || !a->out || (a->batch > 0 && a->max_pages > 0 && !a->page_table)) {
    fat_host::set_error("fat_cache_stats: a required pointer is NULL");
    return FAT_E_INVALID;
  }
  if (a->batch < 0 || a->max_pages < 0 || a->page_size <= 0 || (a->max_pages > 0 && a->page_table_stride < a->max_pages)) {
    fat_host::set_error("fat_cache_stats: batch %d, max_pages %d, page_size %d or page_table_stride %lld invalid",
                        a->batch, a->max_pages, a->page_size, (long long)a->page_table_stride);
    return FAT_E_INVALID;
  }
  hipLaunchKernelGGL(fat::cache_stats_kernel, dim3(1), dim3(fat::kStatsThreads), 0,
                     static_cast<hipStream_t>(stream_ptr), a->seq_lens, a->page_table, a->batch, a->max_pages,
                     a->page_table_stride, a->page_size, a->out);
  return fat_host::launch_status("cache_stats_kernel");
}
