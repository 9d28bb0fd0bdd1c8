// decode_params.h -- the argument block shared by the decode kernels
// (decode.hip: VALU and MFMA decode and the split-K merge; decode_generic.hip:
// the LDS-tiled decode for the shapes the other two do not take).
#pragma once

#include "fat_common.h"

namespace fat {

// Storage of K/V relative to the query type: the same 16/32-bit type, or
// 8-bit codes with one fp32 scale per (page, KV head).
enum KvKind { KV_SAME = 0, KV_I8 = 1, KV_FP8 = 2 };

struct DecodeParams {
  const uint8_t* q;
  const uint8_t* k;
  const uint8_t* v;
  const float* ks;
  const float* vs;
  const int32_t* pt;
  const int32_t* lens;
  uint8_t* out;
  float* ws_acc;  // [B, H, S, D]
  float* ws_ml;   // [B, H, S, 2]  (m in log2 units, l)
  // Split-K tickets, one per (sequence, workgroup row) = gridDim.y * B; NULL:
  // the partitions are merged by decode_merge_kernel in a second launch.
  int32_t* ctr;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sp, k_ss, k_sh;
  int64_t v_sp, v_ss, v_sh;
  int64_t sc_sp, sc_sh;
  int64_t pt_sb;
  int64_t o_sb, o_sh, o_st;
  int32_t H, Hkv, group, hg_per_kv;
  int32_t T;  // query tokens per sequence (1 = single-query decode)
  int32_t P, log2P, num_pages, max_pages;  // log2P = -1: page_size not a power of two
  int32_t pps_fixed;  // pages per partition, 0 = ceil(np / split_k)
  float scale_log2;  // softmax_scale * log2(e)
};

// ---------------------------------------------------------------------------
// Split-K merge inside the decode launch.  Every partition workgroup of a
// (sequence b, workgroup row y) stores its (acc, m, l) rows to the workspace
// and then draws a ticket from ctr[b * gridDim.y + y]; the workgroup that
// draws split_k - 1 is the last one to finish, merges the rows of every
// partition by log-sum-exp (decode.py:316-356 semantics: M = max_s m_s,
// o = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M)) and puts the ticket
// counter back to 0.  The counters are therefore zero again once a launch
// completes, for the next launch and for graph replays.
// Ordering: every thread fences (agent scope: its stores leave this XCD's L2
// before the ticket is drawn) before the barrier that precedes the ticket;
// the last workgroup fences again before reading the other partitions'
// rows.  The ticket is a global vector atomic.
// rows: the (token, head) rows the workgroup covers; row_th(r, t, h) names
// row r.  Called by every thread of the workgroup, after its partial
// stores; nothing may follow it in the kernel.
// ---------------------------------------------------------------------------
constexpr int kMergeChunk = 16;  // partitions whose loads are issued together

template <typename QT, typename RowFn>
__device__ __forceinline__ void merge_partitions_if_last(const DecodeParams& p, int b, int S, int D, int nrows,
                                                         RowFn row_th) {
  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t* ctr = p.ctr + (int64_t)b * gridDim.y + blockIdx.y;
    const int ticket = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    const int last = ticket == S - 1;
    if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int nt = blockDim.x;
  for (int idx = threadIdx.x; idx < nrows * D; idx += nt) {
    const int r = idx / D;
    const int d = idx - r * D;
    int t, h;
    row_th(r, t, h);
    const int64_t row0 = (((int64_t)b * p.T + t) * p.H + h) * S;
    const float* ml = p.ws_ml + row0 * 2;
    const float* ac = p.ws_acc + row0 * D + d;
    // M over every partition first (one extra round of loads beyond 16
    // partitions), then the weighted sums in partition order: the same
    // arithmetic as decode_merge_kernel, so both merges give the same bits.
    float M = -INFINITY;
    if (S > kMergeChunk) {
      for (int s0 = 0; s0 < S; s0 += kMergeChunk) {
#pragma unroll
        for (int j = 0; j < kMergeChunk; ++j) M = fmaxf(M, s0 + j < S ? ml[2 * min(s0 + j, S - 1)] : -INFINITY);
      }
    }
    float A = 0.f, L = 0.f;
    for (int s0 = 0; s0 < S; s0 += kMergeChunk) {
      float m[kMergeChunk], l[kMergeChunk], a[kMergeChunk];
#pragma unroll
      for (int j = 0; j < kMergeChunk; ++j) {
        const int sc = min(s0 + j, S - 1);  // past S: re-read the last partition, weight 0 below
        m[j] = ml[2 * sc];
        l[j] = ml[2 * sc + 1];
        a[j] = ac[(int64_t)sc * D];
      }
#pragma unroll
      for (int j = 0; j < kMergeChunk; ++j) {
        if (s0 + j >= S) {
          m[j] = -INFINITY;
          l[j] = 0.f;
          a[j] = 0.f;
        }
      }
      if (S <= kMergeChunk) {
#pragma unroll
        for (int j = 0; j < kMergeChunk; ++j) M = fmaxf(M, m[j]);
      }
      if (M == -INFINITY) break;  // no partition saw a key
#pragma unroll
      for (int j = 0; j < kMergeChunk; ++j) {
        const float f = fast_exp2(m[j] - M);  // 0 for padded or empty partitions
        A = __builtin_fmaf(a[j], f, A);
        L = __builtin_fmaf(l[j], f, L);
      }
    }
    store_elem<QT>(p.out, (int64_t)b * p.o_sb + (int64_t)t * p.o_st + (int64_t)h * p.o_sh + d,
                   L > 0.f ? A / L : 0.f);
  }
}

}  // namespace fat

namespace fat_host {

// Heads of one GQA group that a workgroup of the generic decode holds.
constexpr int kGenericHeads = 8;

// Launch the generic decode (decode_generic.hip) on `grid` = (split_k,
// num_kv_heads * ceil(group / heads_per_wg), batch); q_dtype is a fat_dtype.
// Returns FAT_OK or FAT_E_UNSUPPORTED / FAT_E_LAUNCH with the error set.
int launch_decode_generic(const fat::DecodeParams& prm, int q_dtype, int kv, int head_dim, int heads_per_wg,
                          dim3 grid, hipStream_t stream);

}  // namespace fat_host
