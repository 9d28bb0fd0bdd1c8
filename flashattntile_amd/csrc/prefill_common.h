// prefill_common.h -- what the prefill kernels of prefill.hip and
// prefill_wide.hip share: the launch parameters, the tile constants, the
// lazy-rescale bounds of the ping-pong kernels and the epilogue that writes
// a wave's output rows through LDS.
#pragma once

#include "fat_common.h"

namespace fat {

struct PrefillParams {
  const uint8_t* q;
  const uint8_t* k;
  const uint8_t* v;
  const int32_t* cu_q;
  const int32_t* cu_k;
  uint8_t* out;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;  // element strides (k/v_st: slot stride when paged)
  int32_t B, H, Hkv, group, nqb;
  float scale_log2;  // > 0 (or NaN): the kernels fold it into the exponent's fma
  // Applied to every Q dword as it is loaded, (q & q_and) ^ q_xor: a
  // negative softmax scale runs as |scale| with Q's signs flipped (exact),
  // a zero scale with Q zeroed (every logit 0).  Identity: ~0u, 0.
  uint32_t q_and, q_xor;
  // Paged K/V (PAGED instantiations only).
  const int32_t* pt;    // page table [B, max_pages]
  const int32_t* lens;  // kv_len per sequence
  int64_t pt_sb;        // page-table row stride
  int64_t k_sp, v_sp;   // page strides (elements)
  int32_t pshift;       // log2(page_size)
  int32_t num_pages, max_pages;
  // bf16 V converted ahead of the kernel (VPRE instantiations): v points at
  // fp16 values scaled by 2^-v_head_scale[sequence * Hkv + kv head].
  const int32_t* v_head_scale;
  // Wide kernel: > 0 when the launch's nqb * B work items (query block,
  // sequence) run longest causal chain first (ranked on the device); 0: in
  // block order.
  int32_t rank_items;
};

constexpr int kBM = 128;
// Query rows per workgroup of the 64-rows-per-wave kernel (prefill_wide.hip).
constexpr int kWideBM = 512;
// Most sequences a wide launch ranks its work items over (the ranking costs
// each thread a loop over the sequences; one item per thread, so at most
// kWideBM items).
constexpr int kWideRankMaxSeqs = 16;
constexpr int kBN = 64;

// Lazy-rescale bound of the ping-pong kernel (log2 units) and the partial
// row-sum level above which its exact softmax path runs.
constexpr float kLazyPP = 15.0f;
constexpr float kLazyPPSum = 32768.0f;  // 2^kLazyPP

// Epilogue of a wave that owns 32 query rows (row0 ..): O = acc / l (times
// 2^e_acc for bf16) to the output, through `ob`, an LDS area of
// kOutStage<D> elements (32 rows of D + 8) that no other wave touches
// meanwhile: the wave writes its O^T fragments there as T, then each lane
// stores 16 contiguous bytes of a row (8-byte pieces when the output rows
// are not 16-byte aligned).
template <int D> constexpr int kOutStage = 32 * (D + 8);
template <typename T, int D, int DB>
__device__ __forceinline__ void write_rows_via_lds(uint16_t* ob, int li, int g, int lane, const f32x16 (&acc)[DB],
                                                   float l_run, int e_acc, bool vh, const PrefillParams& p,
                                                   int q_start, int q_len, int h, int row0) {
  constexpr int OS = D + 8;  // row stride (elements)
  const float l_tot = xor32<OpAdd>(l_run);
  float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (vh) inv *= as_f32((u32)(127 + e_acc) << 23);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int d0 = 32 * db + 4 * g + 8 * rr;
      u32x2 pk;
      pk[0] = Pair<T>::pack(acc[db][4 * rr + 0] * inv, acc[db][4 * rr + 1] * inv);
      pk[1] = Pair<T>::pack(acc[db][4 * rr + 2] * inv, acc[db][4 * rr + 3] * inv);
      *reinterpret_cast<u32x2*>(&ob[li * OS + d0]) = pk;
    }
  wave_lds_fence();
  constexpr int CPR_O = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR_O;  // rows per store instruction
  const int oc = lane % CPR_O;
  const int orow = lane / CPR_O;
  const bool o16 = ((reinterpret_cast<uintptr_t>(p.out) | (uintptr_t)(2 * p.o_st) | (uintptr_t)(2 * p.o_sh)) & 15) == 0;
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = i * RPI + orow;
    const u32x4 val = *reinterpret_cast<const u32x4*>(&ob[r * OS + 8 * oc]);
    if ((unsigned)(row0 + r) < (unsigned)q_len) {  // rows in [0, q_len)
      uint8_t* dst = p.out + 2 * ((int64_t)(q_start + row0 + r) * p.o_st + (int64_t)h * p.o_sh + 8 * oc);
      if (o16) {
        *reinterpret_cast<u32x4*>(dst) = val;
      } else {
        *reinterpret_cast<u32x2*>(dst) = u32x2{val[0], val[1]};
        *reinterpret_cast<u32x2*>(dst + 8) = u32x2{val[2], val[3]};
      }
    }
  }
}

}  // namespace fat

namespace fat_host {
// The 8-wave prefill kernel with 64 query rows per wave (prefill_wide.hip)
// for packed fp16, or packed bf16 whose V was converted to fp16 ahead of the
// kernel (prm.v / v_head_scale), at head_dim 128.  `grid` counts blocks of
// fat::kWideBM query rows.
int launch_prefill_wide(const fat::PrefillParams& prm, bool bf16, bool causal, dim3 grid, hipStream_t stream);
// The generic VALU prefill (prefill_generic.hip) for a fat_dtype and a
// power-of-two head_dim 16..512, packed or paged; `grid` counts blocks of 32
// query rows.
int launch_prefill_generic(const fat::PrefillParams& prm, int dtype, int D, bool causal, bool paged, dim3 grid,
                           hipStream_t stream);
// Packed copies of a paged launch's K/V rows (prefill_stage.hip): cu_k
// [B + 1] from `paged`.lens clamped to `cap`, then every sequence's rows into
// kdst / vdst as [cu_k[B], Hkv, D] (2-byte elements, head_dim 128).
int launch_paged_stage(const fat::PrefillParams& paged, int D, int B, int cap, int32_t* cu_k, uint8_t* kdst,
                       uint8_t* vdst, hipStream_t stream);
}  // namespace fat_host
