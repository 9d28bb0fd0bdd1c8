// prefill_generic.hip -- varlen prefill for the shapes the MFMA prefill
// kernels (prefill.hip, prefill_wide.hip) do not take: fp32 inputs, and
// head_dim 16 or 512 (every power of two from 16 to 512 runs here when forced).
//
// Semantics are those of the other prefill kernels and of the reference's
// _fwd_varlen_kernel (flashattn_tile/kernels/prefill.py:35-138): per (query
// block, query head, sequence) an online softmax over the sequence's keys,
// bottom-right causal masking (query i sees key j iff j <= i + kv_len -
// q_len), packed or paged K/V, output in the input dtype.  The reference
// runs fp32 through its fp32 fallback (kernels/prefill.py:286-290); here the
// scores, softmax and PV all stay in fp32, with P not rounded.
//
// Design: one workgroup of 256 threads per block of 32 query rows.
//   * eight threads share a row: thread c of a row holds the row's q and O
//     for dims VEC c + 8 VEC i + e (i < D / (8 VEC), e < VEC; VEC = 4, 2 at
//     D16) in registers, as fp32;
//   * K and V tiles (32 keys, 16 at D >= 256) are loaded 16 bytes per thread
//     and stored in LDS as fp32; every thread of a row reads the same key
//     rows, so a read is one float4 per thread, broadcast to the 32 rows;
//   * a tile's scores are reduced over the row's eight threads with DPP, then
//     the softmax takes the tile max once (rescaling O only when it grows)
//     and PV accumulates over the tile's keys.
// It is a VALU kernel: the fp16/bf16 shapes that the MFMA kernels take stay
// there.
#include "prefill_common.h"

namespace fat {

template <typename T>
struct GElem {
  static constexpr int kBytes = std::is_same<T, F32>::value ? 4 : 2;
  static constexpr int kPerChunk = 16 / kBytes;  // elements per 16-byte load
  // 16 bytes of T as kPerChunk floats.
  static __device__ __forceinline__ void unpack(const u32x4& x, float* f) {
    if constexpr (std::is_same<T, F32>::value) {
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = as_f32(x[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = Pair<T>::lo(x[e]);
        f[2 * e + 1] = Pair<T>::hi(x[e]);
      }
    }
  }
  static __device__ __forceinline__ float load1(const uint8_t* base, int64_t idx) {
    if constexpr (std::is_same<T, F32>::value) return reinterpret_cast<const float*>(base)[idx];
    else return Pair<T>::lo((u32)reinterpret_cast<const uint16_t*>(base)[idx]);
  }
};

// Sum over the eight lanes of a row group (lanes 8k .. 8k + 7).
__device__ __forceinline__ float sum8(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  x += dpp<kDppHalfMirror>(x);
  return x;
}

template <typename T, int D, bool CAUSAL, int PG>
__global__ __launch_bounds__(256) void prefill_generic_kernel(const PrefillParams p) {
  constexpr int BM = 32;                   // query rows per workgroup
  constexpr int TK = D >= 256 ? 16 : 32;   // keys per tile
  constexpr int VEC = D >= 32 ? 4 : 2;     // consecutive dims per thread group
  constexpr int NG = D / (8 * VEC);        // dim groups per thread
  constexpr int EPC = GElem<T>::kPerChunk;
  constexpr int CPR = D / EPC;             // 16-byte chunks per K/V row
  constexpr int RS = D + 4;                // LDS row stride (floats)
  static_assert(NG >= 1 && NG * 8 * VEC == D, "head_dim must be a power of two in [16, 512]");
  static_assert(CPR >= 1, "head_dim too small for 16-byte loads");
  __shared__ __attribute__((aligned(16))) float sK[TK * RS];
  __shared__ __attribute__((aligned(16))) float sV[TK * RS];

  const int per = p.B * p.H;
  const int outer = blockIdx.x / per;
  const int rem = blockIdx.x - outer * per;
  const int b = rem / p.H;
  const int j = rem - b * p.H;
  const int kvh = j % p.Hkv;
  const int h = kvh * p.group + j / p.Hkv;
  const int mb = p.nqb - 1 - outer;

  const int q_start = p.cu_q[b];
  const int q_len = p.cu_q[b + 1] - q_start;
  constexpr bool PAGED = PG != 0;
  const int k_start = PAGED ? 0 : p.cu_k[b];
  const int kv_len = PAGED ? min(max(p.lens[b], 0), p.max_pages << p.pshift) : p.cu_k[b + 1] - k_start;
  if (mb * BM >= q_len) return;  // uniform over the workgroup

  const int tid = threadIdx.x;
  const int r = tid >> 3;  // query row of this thread in the block
  const int c = tid & 7;   // its part of the row
  const int row = mb * BM + r;
  const int shift = kv_len - q_len;
  constexpr int EB = GElem<T>::kBytes;

  float q[NG][VEC];
  {
    const int qr = min(row, q_len - 1);
    const int64_t qb = (int64_t)(q_start + qr) * p.q_st + (int64_t)h * p.q_sh;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) q[i][e] = GElem<T>::load1(p.q, qb + 8 * VEC * i + VEC * c + e);
  }
  float acc[NG][VEC];
#pragma unroll
  for (int i = 0; i < NG; ++i)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[i][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float cl = p.scale_log2;  // softmax_scale * log2(e)

  int hi = kv_len;
  if (CAUSAL) hi = min(kv_len, (mb + 1) * BM + shift);
  const int n_tiles = hi > 0 ? (hi + TK - 1) / TK : 0;
  const int32_t* ptrow = PAGED ? p.pt + (int64_t)b * p.pt_sb : nullptr;
  const int pmask = PAGED ? (1 << p.pshift) - 1 : 0;

  for (int t = 0; t < n_tiles; ++t) {
    const int n0 = t * TK;
    __syncthreads();  // the previous tile's reads are done
    for (int idx = tid; idx < TK * CPR; idx += 256) {
      const int kr = idx / CPR;
      const int ch = idx - kr * CPR;
      const int key = n0 + kr;
      float fk[EPC], fv[EPC];
      if (key < kv_len) {
        int64_t ko, vo;
        if constexpr (PAGED) {
          const int page = min(max(ptrow[key >> p.pshift], 0), p.num_pages - 1);
          const int slot = key & pmask;
          ko = (int64_t)page * p.k_sp + (int64_t)slot * p.k_st + (int64_t)kvh * p.k_sh;
          vo = (int64_t)page * p.v_sp + (int64_t)slot * p.v_st + (int64_t)kvh * p.v_sh;
        } else {
          ko = (int64_t)(k_start + key) * p.k_st + (int64_t)kvh * p.k_sh;
          vo = (int64_t)(k_start + key) * p.v_st + (int64_t)kvh * p.v_sh;
        }
        GElem<T>::unpack(*reinterpret_cast<const u32x4*>(p.k + EB * (ko + EPC * ch)), fk);
        GElem<T>::unpack(*reinterpret_cast<const u32x4*>(p.v + EB * (vo + EPC * ch)), fv);
      } else {  // past the sequence: zeros (masked scores; finite V)
#pragma unroll
        for (int e = 0; e < EPC; ++e) fk[e] = fv[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < EPC; e += 4) {
        *reinterpret_cast<f32x4*>(&sK[kr * RS + EPC * ch + e]) = f32x4{fk[e], fk[e + 1], fk[e + 2], fk[e + 3]};
        *reinterpret_cast<f32x4*>(&sV[kr * RS + EPC * ch + e]) = f32x4{fv[e], fv[e + 1], fv[e + 2], fv[e + 3]};
      }
    }
    __syncthreads();

    // Scores of the tile's keys for this row (log2 units), masked.
    const int lim = CAUSAL ? min(kv_len - 1, row + shift) : kv_len - 1;
    float s[TK];
    float tmax = -INFINITY;
#pragma unroll
    for (int k = 0; k < TK; ++k) {
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        const float* kp = &sK[k * RS + 8 * VEC * i + VEC * c];
        if constexpr (VEC == 4) {
          const f32x4 kv4 = *reinterpret_cast<const f32x4*>(kp);
#pragma unroll
          for (int e = 0; e < 4; ++e) part = __builtin_fmaf(q[i][e], kv4[e], part);
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) part = __builtin_fmaf(q[i][e], kp[e], part);
        }
      }
      const float sc = sum8(part) * cl;
      s[k] = (n0 + k) <= lim ? sc : -INFINITY;
      tmax = fmaxf(tmax, s[k]);
    }
    // Online softmax: O and l move only when the tile raises the row max.
    if (tmax > m_run) {
      const float alpha = fast_exp2(m_run - tmax);  // 0 while m_run is -inf
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[i][e] *= alpha;
      m_run = tmax;
    }
    if (m_run == -INFINITY) continue;  // no visible key yet (this row)
#pragma unroll
    for (int k = 0; k < TK; ++k) {
      const float pk = fast_exp2(s[k] - m_run);
      l_run += pk;
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        const float* vp = &sV[k * RS + 8 * VEC * i + VEC * c];
        if constexpr (VEC == 4) {
          const f32x4 vv4 = *reinterpret_cast<const f32x4*>(vp);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][e] = __builtin_fmaf(pk, vv4[e], acc[i][e]);
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[i][e] = __builtin_fmaf(pk, vp[e], acc[i][e]);
        }
      }
    }
  }

  if (row < q_len) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    const int64_t ob = (int64_t)(q_start + row) * p.o_st + (int64_t)h * p.o_sh;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) store_elem<T>(p.out, ob + 8 * VEC * i + VEC * c + e, acc[i][e] * inv);
  }
}

}  // namespace fat

namespace fat_host {

template <typename T, int D, int PG>
static void launch_generic_d(const fat::PrefillParams& prm, bool causal, dim3 grid, hipStream_t stream) {
  if (causal) hipLaunchKernelGGL((fat::prefill_generic_kernel<T, D, true, PG>), grid, dim3(256), 0, stream, prm);
  else hipLaunchKernelGGL((fat::prefill_generic_kernel<T, D, false, PG>), grid, dim3(256), 0, stream, prm);
}

template <typename T, int PG>
static int launch_generic_t(const fat::PrefillParams& prm, int D, bool causal, dim3 grid, hipStream_t stream) {
  switch (D) {
    case 16: launch_generic_d<T, 16, PG>(prm, causal, grid, stream); break;
    case 32: launch_generic_d<T, 32, PG>(prm, causal, grid, stream); break;
    case 64: launch_generic_d<T, 64, PG>(prm, causal, grid, stream); break;
    case 128: launch_generic_d<T, 128, PG>(prm, causal, grid, stream); break;
    case 256: launch_generic_d<T, 256, PG>(prm, causal, grid, stream); break;
    case 512: launch_generic_d<T, 512, PG>(prm, causal, grid, stream); break;
    default:
      set_error("prefill: head_dim %d unsupported (a power of two from 16 to 512)", D);
      return FAT_E_UNSUPPORTED;
  }
  return launch_status("prefill_generic_kernel");
}

int launch_prefill_generic(const fat::PrefillParams& prm, int dtype, int D, bool causal, bool paged, dim3 grid,
                           hipStream_t stream) {
  if (dtype == FAT_DTYPE_F32)
    return paged ? launch_generic_t<fat::F32, 1>(prm, D, causal, grid, stream)
                 : launch_generic_t<fat::F32, 0>(prm, D, causal, grid, stream);
  if (dtype == FAT_DTYPE_BF16)
    return paged ? launch_generic_t<fat::BF16, 1>(prm, D, causal, grid, stream)
                 : launch_generic_t<fat::BF16, 0>(prm, D, causal, grid, stream);
  return paged ? launch_generic_t<fat::F16, 1>(prm, D, causal, grid, stream)
               : launch_generic_t<fat::F16, 0>(prm, D, causal, grid, stream);
}

}  // namespace fat_host
