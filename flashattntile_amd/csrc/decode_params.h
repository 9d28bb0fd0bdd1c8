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
  // Split-K merge inside the decode launch: one counter per (sequence, head
  // group) = blockIdx.z * gridDim.y + blockIdx.y, zero between launches;
  // nullptr: a second kernel merges.  smax: the merge's unrolled partition
  // count (a power of two >= split_k, at most 16).
  int32_t* counters;
  int32_t smax;
};

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
