// prefill_stage.hip -- packed copies of the K/V rows of a paged prefill
// launch, so that long paged chunks run on the packed wide kernel
// (prefill_wide.hip).
//
// A paged prefill chunk whose sequences average thousands of queries is
// compute-bound: each key row is read by every query block of its sequence,
// while staging reads and writes it once.  The copies are dense
// [total_k, Hkv, D] arrays in the launch's workspace, in sequence order, with
// the sequences' offsets cu_k computed on the device from seq_lens.  The
// paged semantics are kept: kv_len = clamp(seq_lens[b], 0, max_pages *
// page_size) and page ids are clamped to [0, num_pages), as in the paged
// kernels (a bad table gives a wrong answer, never an out-of-bounds read).
#include "prefill_common.h"

namespace fat {

// Key rows one staging workgroup copies (every KV head, K and V).
constexpr int kStageRows = 16;

// cu_k[0] = 0, cu_k[b + 1] = cu_k[b] + clamp(lens[b], 0, cap).  One
// workgroup of 1024 threads scans the lengths 1024 at a time.
__global__ __launch_bounds__(1024) void paged_stage_offsets_kernel(const int32_t* __restrict__ lens, int B, int cap,
                                                                   int32_t* __restrict__ cu_k) {
  __shared__ int wsum[16];
  __shared__ int carry;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  if (tid == 0) {
    carry = 0;
    cu_k[0] = 0;
  }
  __syncthreads();
  for (int base = 0; base < B; base += 1024) {
    const int i = base + tid;
    int x = i < B ? min(max(lens[i], 0), cap) : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off);
      if (lane >= off) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int pre = carry;
    for (int j = 0; j < w; ++j) pre += wsum[j];
    if (i < B) cu_k[i + 1] = pre + x;
    __syncthreads();  // every thread has read carry and wsum
    if (tid == 1023) carry = pre + x;
    __syncthreads();
  }
}

// Rows [kStageRows x, kStageRows (x + 1)) of sequence y: every KV head's K
// and V row to kdst / vdst at row cu_k[y] + key.  16-byte chunks; a head row
// is D / 8 chunks, a key row Hkv of them, contiguous in the copies.
template <int D>
__global__ __launch_bounds__(256) void paged_stage_kv_kernel(const PrefillParams p, const int32_t* __restrict__ cu_k,
                                                             uint8_t* __restrict__ kdst, uint8_t* __restrict__ vdst) {
  constexpr int CPH = D / 8;  // chunks per head row (2-byte elements)
  const int b = blockIdx.y;
  const int s0 = cu_k[b];
  const int len = cu_k[b + 1] - s0;
  const int key0 = blockIdx.x * kStageRows;
  if (key0 >= len) return;
  const int nrows = min(kStageRows, len - key0);
  const int cpr = p.Hkv * CPH;
  const int32_t* ptrow = p.pt + (int64_t)b * p.pt_sb;
  const int pmask = (1 << p.pshift) - 1;
  for (int c = threadIdx.x; c < nrows * cpr; c += 256) {
    const int r = c / cpr;
    const int rc = c - r * cpr;
    const int h = rc / CPH;
    const int ch = rc - h * CPH;
    const int key = key0 + r;
    const int page = min(max(ptrow[key >> p.pshift], 0), p.num_pages - 1);
    const int slot = key & pmask;
    const int64_t ko = (int64_t)page * p.k_sp + (int64_t)slot * p.k_st + (int64_t)h * p.k_sh + 8 * ch;
    const int64_t vo = (int64_t)page * p.v_sp + (int64_t)slot * p.v_st + (int64_t)h * p.v_sh + 8 * ch;
    const int64_t d = ((int64_t)(s0 + key) * p.Hkv + h) * D + 8 * ch;
    const u32x4 kx = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.k + 2 * ko));  // read once
    const u32x4 vx = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.v + 2 * vo));
    *reinterpret_cast<u32x4*>(kdst + 2 * d) = kx;
    *reinterpret_cast<u32x4*>(vdst + 2 * d) = vx;
  }
}

}  // namespace fat

namespace fat_host {

int launch_paged_stage(const fat::PrefillParams& paged, int D, int B, int cap, int32_t* cu_k, uint8_t* kdst,
                       uint8_t* vdst, hipStream_t stream) {
  if (D != 128) {
    set_error("prefill staging: head_dim %d (128 only)", D);
    return FAT_E_UNSUPPORTED;
  }
  hipLaunchKernelGGL(fat::paged_stage_offsets_kernel, dim3(1), dim3(1024), 0, stream, paged.lens, B, cap, cu_k);
  const int rc = launch_status("paged_stage_offsets_kernel");
  if (rc != FAT_OK) return rc;
  const dim3 grid((unsigned)((cap + fat::kStageRows - 1) / fat::kStageRows), (unsigned)B);
  hipLaunchKernelGGL((fat::paged_stage_kv_kernel<128>), grid, dim3(256), 0, stream, paged, cu_k, kdst, vdst);
  return launch_status("paged_stage_kv_kernel");
}

}  // namespace fat_host
