// kvwrite.hip -- the paged KV-cache write path on gfx950: per-(page, KV head)
// quantisation of pages, and the one-token-per-sequence append with an
// optional int8/fp8 copy of the cache that is requantised where it changed.
//
// Semantics follow the FlashAttnTile data contract:
//   flashattn_tile/quant.py:84-142   quantize_kv_pages: per (page, KV head)
//       scale = max(absmax over (slot, dim) / {127 | 448}, 1e-8);
//       int8 = clamp(round_half_even(x / scale), -127, 127);
//       fp8  = e4m3fn(clamp(x / scale, -448, 448));
//   flashattn_tile/paging.py:172-210 append_tokens: token b goes to position
//       seq_lens[b] through the page table, then seq_lens += 1.
// A page's scale depends on every slot of that page, so appending to a
// quantised cache means requantising each touched (page, KV head) from the
// full-precision page; done here for exactly the touched pages, it gives the
// bytes a quantisation of the whole updated cache would give.
//
// Work split: one wave per (page, KV head) unit.  A unit is page_size rows of
// head_dim elements at a stride of num_kv_heads * head_dim.  Lanes load it in
// 16-byte chunks -- all of them at once and kept in registers when the unit
// is at most 512 chunks (8 KiB of fp16: page_size * head_dim <= 4096), else in
// two passes whose second is an L2 hit -- reduce the absmax with DPP and
// permlane, and store 8 (fp16/bf16 source) or 4 (fp32 source) codes per lane.
// When a stride or pointer is not 16-byte aligned the same kernels run one
// element per lane.  HBM-bound byte work: no MFMA.
#include <math.h>

#include <initializer_list>
#include <type_traits>

#include "fat_common.h"

namespace fat {

template <typename S> struct SrcBytes { static constexpr int kValue = 2; };
template <> struct SrcBytes<F32> { static constexpr int kValue = 4; };

enum QuantKind { Q_I8 = 0, Q_FP8 = 1 };

template <int QK> struct QMax;
template <> struct QMax<Q_I8> { static constexpr float kValue = 127.0f; };
template <> struct QMax<Q_FP8> { static constexpr float kValue = 448.0f; };
constexpr float kQuantMinScale = 1e-8f;

// One source element as float.
template <typename S>
__device__ __forceinline__ float load_one(const uint8_t* p) {
  if constexpr (std::is_same_v<S, F32>) return *reinterpret_cast<const float*>(p);
  else if constexpr (std::is_same_v<S, F16>) return (float)*reinterpret_cast<const f16*>(p);
  else return as_f32((u32)*reinterpret_cast<const uint16_t*>(p) << 16);
}

// The CH source values held in one 16-byte chunk, as floats.
template <typename S, int CH>
__device__ __forceinline__ void unpack_chunk(const u32x4& w, float (&f)[CH]) {
  if constexpr (std::is_same_v<S, F32>) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = as_f32(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = Pair<S>::lo(w[i]);
      f[2 * i + 1] = Pair<S>::hi(w[i]);
    }
  }
}

// CH consecutive source elements as floats (CH > 1: one 16-byte load).
template <typename S, int CH>
__device__ __forceinline__ void load_chunk(const uint8_t* p, float (&f)[CH]) {
  if constexpr (CH == 1) f[0] = load_one<S>(p);
  else unpack_chunk<S, CH>(*reinterpret_cast<const u32x4*>(p), f);
}

// x / scale, rounded as the correctly rounded fp32 division would round it
// for the purpose of quantisation.  fp32 sources use the division itself.
// 16-bit sources use q = x * r with r = 1 / scale (correctly rounded) and one
// fma correction, q += (x - q * scale) * r, with x's sign put back (the
// correction turns -0 into +0).  This was checked against the division by
// exhaustion over every pair (absmax, x) of fp16 values and every pair of
// bf16 values, for both qmax = 127 and 448 -- 2^32 pairs each, only the
// |x| <= absmax a unit can hold: fp16 quotients are bit-identical; bf16
// quotients differ only for fp32-denormal inputs, and the int8 and fp8 codes
// never differ.
template <typename S>
__device__ __forceinline__ float scaled(float x, float sc, float r) {
  if constexpr (std::is_same_v<S, F32>) {
    return x / sc;
  } else {
    const float q = x * r;
    const float e = fmaf(-q, sc, x);
    return __builtin_copysignf(fmaf(e, r, q), x);
  }
}

// Code of one scaled value y, in the low byte.
template <int QK>
__device__ __forceinline__ u32 quant_code(float y) {
  if constexpr (QK == Q_I8) {
    // v_rndne_f32 (round half to even, as torch.round), then v_med3_f32.
    const float r = __builtin_amdgcn_fmed3f(__builtin_rintf(y), -127.0f, 127.0f);
    return (u32)(int)r & 0xffu;
  } else {
    const float c = __builtin_amdgcn_fmed3f(y, -448.0f, 448.0f);
    // v_cvt_pk_fp8_f32: OCP e4m3fn, round to nearest even.
    return (u32)__builtin_amdgcn_cvt_pk_fp8_f32(c, c, 0, false) & 0xffu;
  }
}

// Four codes packed little-endian in one dword.
template <int QK>
__device__ __forceinline__ u32 quant_code4(float a, float b, float c, float d) {
  if constexpr (QK == Q_I8) {
    return quant_code<QK>(a) | (quant_code<QK>(b) << 8) | (quant_code<QK>(c) << 16) | (quant_code<QK>(d) << 24);
  } else {
    const float a1 = __builtin_amdgcn_fmed3f(a, -448.0f, 448.0f), b1 = __builtin_amdgcn_fmed3f(b, -448.0f, 448.0f);
    const float c1 = __builtin_amdgcn_fmed3f(c, -448.0f, 448.0f), d1 = __builtin_amdgcn_fmed3f(d, -448.0f, 448.0f);
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a1, b1, 0, false);
    return (u32)__builtin_amdgcn_cvt_pk_fp8_f32(c1, d1, lo, true);
  }
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<kDppXor1>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  x = fmaxf(x, dpp<kDppRor4>(x));
  x = fmaxf(x, dpp<kDppRor8>(x));
  x = xor16<OpMax>(x);
  x = xor32<OpMax>(x);
  return x;
}

// Codes of the CH source values `f` stored at o (CH bytes).
template <typename S, int QK, int CH>
__device__ __forceinline__ void store_codes(uint8_t* o, const float (&f)[CH], float sc, float r) {
  if constexpr (CH == 1) {
    *o = (uint8_t)quant_code<QK>(scaled<S>(f[0], sc, r));
  } else if constexpr (CH == 4) {
    *reinterpret_cast<u32*>(o) = quant_code4<QK>(scaled<S>(f[0], sc, r), scaled<S>(f[1], sc, r),
                                                 scaled<S>(f[2], sc, r), scaled<S>(f[3], sc, r));
  } else {
    u32x2 w;
    w[0] = quant_code4<QK>(scaled<S>(f[0], sc, r), scaled<S>(f[1], sc, r), scaled<S>(f[2], sc, r),
                           scaled<S>(f[3], sc, r));
    w[1] = quant_code4<QK>(scaled<S>(f[4], sc, r), scaled<S>(f[5], sc, r), scaled<S>(f[6], sc, r),
                           scaled<S>(f[7], sc, r));
    *reinterpret_cast<u32x2*>(o) = w;
  }
}

// Per-unit scale from the wave's partial absmax: max(absmax / qmax, 1e-8),
// the division correctly rounded (the HIP default for fp32 '/').
template <int QK>
__device__ __forceinline__ float unit_scale(float amax) {
  return fmaxf(wave_max(amax) / QMax<QK>::kValue, kQuantMinScale);
}

// A unit of n <= 64 * NC 16-byte chunks: every chunk is loaded up front and
// held in registers (raw, 4 VGPRs each), so the page is read once and all of
// a lane's loads are in flight together.
template <typename S, int QK, int CH, int NC>
__device__ __forceinline__ void quantize_unit_regs(const uint8_t* src, int64_t s_ss, uint8_t* dst, int64_t d_ss,
                                                   float* scale, int cpr, int n, int lane) {
  constexpr int ES = SrcBytes<S>::kValue;
  u32x4 raw[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    raw[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < n) {
      const int slot = c / cpr;
      // read once: streaming (nontemporal) load
      raw[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(src + ES * ((int64_t)slot * s_ss + (c - slot * cpr) * CH)));
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float f[CH];
    unpack_chunk<S, CH>(raw[i], f);
#pragma unroll
    for (int j = 0; j < CH; ++j) amax = fmaxf(amax, fabsf(f[j]));
  }
  const float sc = unit_scale<QK>(amax);
  const float r = 1.0f / sc;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    if (c < n) {
      const int slot = c / cpr;
      float f[CH];
      unpack_chunk<S, CH>(raw[i], f);
      store_codes<S, QK, CH>(dst + (int64_t)slot * d_ss + (c - slot * cpr) * CH, f, sc, r);
    }
  }
  if (lane == 0) *scale = sc;
}

// Any unit size: two passes over the unit (the second an L2 hit).
template <typename S, int QK, int CH>
__device__ __forceinline__ void quantize_unit_loop(const uint8_t* src, int64_t s_ss, uint8_t* dst, int64_t d_ss,
                                                   float* scale, int cpr, int n, int lane) {
  constexpr int ES = SrcBytes<S>::kValue;
  float amax = 0.f;
  for (int c = lane; c < n; c += 64) {
    const int slot = c / cpr;
    float f[CH];
    load_chunk<S, CH>(src + ES * ((int64_t)slot * s_ss + (c - slot * cpr) * CH), f);
#pragma unroll
    for (int i = 0; i < CH; ++i) amax = fmaxf(amax, fabsf(f[i]));
  }
  const float sc = unit_scale<QK>(amax);
  const float r = 1.0f / sc;
  for (int c = lane; c < n; c += 64) {
    const int slot = c / cpr;
    const int d = (c - slot * cpr) * CH;
    float f[CH];
    load_chunk<S, CH>(src + ES * ((int64_t)slot * s_ss + d), f);
    store_codes<S, QK, CH>(dst + (int64_t)slot * d_ss + d, f, sc, r);
  }
  if (lane == 0) *scale = sc;
}

// Quantise one (page, head) unit held by the calling wave.  Element
// (slot, d) is at src + ES * (slot * s_ss + d); its code goes to
// dst[slot * d_ss + d] and the scale to *scale.  VEC: 16-byte chunks (the
// caller checked alignment), else one element per lane.
template <typename S, int QK, bool VEC>
__device__ __forceinline__ void quantize_unit(const uint8_t* src, int64_t s_ss, uint8_t* dst, int64_t d_ss,
                                              float* scale, int P, int D, int lane) {
  if constexpr (VEC) {
    constexpr int CH = 16 / SrcBytes<S>::kValue;
    const int cpr = D / CH;
    const int n = P * cpr;
    if (n <= 64) quantize_unit_regs<S, QK, CH, 1>(src, s_ss, dst, d_ss, scale, cpr, n, lane);
    else if (n <= 128) quantize_unit_regs<S, QK, CH, 2>(src, s_ss, dst, d_ss, scale, cpr, n, lane);
    else if (n <= 256) quantize_unit_regs<S, QK, CH, 4>(src, s_ss, dst, d_ss, scale, cpr, n, lane);
    else if (n <= 512) quantize_unit_regs<S, QK, CH, 8>(src, s_ss, dst, d_ss, scale, cpr, n, lane);
    else quantize_unit_loop<S, QK, CH>(src, s_ss, dst, d_ss, scale, cpr, n, lane);
  } else {
    quantize_unit_loop<S, QK, 1>(src, s_ss, dst, d_ss, scale, D, P * D, lane);
  }
}

struct QuantParams {
  const uint8_t* src;
  uint8_t* dst;
  float* scale;
  int64_t s_sp, s_ss, s_sh;  // source strides (elements)
  int64_t d_sp, d_ss, d_sh;  // code strides
  int64_t c_sp, c_sh;        // scale strides
  int32_t num_pages, P, Hkv, D;
};

// Four waves per workgroup, one (page, head) unit per wave.
template <typename S, int QK, bool VEC>
__global__ __launch_bounds__(256) void quantize_pages_kernel(const QuantParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= (int64_t)p.num_pages * p.Hkv) return;  // whole wave
  const int page = (int)(unit / p.Hkv);
  const int head = (int)(unit - (int64_t)page * p.Hkv);
  constexpr int ES = SrcBytes<S>::kValue;
  quantize_unit<S, QK, VEC>(p.src + ES * ((int64_t)page * p.s_sp + (int64_t)head * p.s_sh), p.s_ss,
                           p.dst + (int64_t)page * p.d_sp + (int64_t)head * p.d_sh, p.d_ss,
                           p.scale + (int64_t)page * p.c_sp + (int64_t)head * p.c_sh, p.P, p.D, lane);
}

struct AppendParams {
  const uint16_t* nk;
  const uint16_t* nv;
  uint16_t* kc;
  uint16_t* vc;
  uint8_t* qk;
  uint8_t* qv;
  float* ks;
  float* vs;
  const int32_t* pt;
  int32_t* lens;
  int64_t nk_sb, nk_sh, nv_sb, nv_sh;
  int64_t k_sp, k_ss, k_sh, v_sp, v_ss, v_sh;
  int64_t qk_sp, qk_ss, qk_sh, qv_sp, qv_ss, qv_sh;
  int64_t sc_sp, sc_sh;
  int64_t pt_sb;
  int32_t batch, Hkv, D, P, num_pages, max_pages;
  int32_t advance;
};

// Physical page and slot of sequence b's next token; false when the position
// or the page id is out of range (the entry is then skipped).
__device__ __forceinline__ bool append_target(const AppendParams& p, int b, int& pos, int& page, int& slot) {
  pos = p.lens[b];
  if (pos < 0 || pos >= p.max_pages * p.P) return false;
  page = p.pt[(int64_t)b * p.pt_sb + pos / p.P];
  slot = pos % p.P;
  return page >= 0 && page < p.num_pages;
}

// One workgroup per sequence: write the K and V rows of every KV head.  When
// no quantised copy follows, advance seq_lens once every thread has read it.
__global__ __launch_bounds__(256) void append_scatter_kernel(const AppendParams p, int advance_here) {
  const int b = blockIdx.x;
  int pos, page, slot;
  const bool ok = append_target(p, b, pos, page, slot);
  if (ok) {
    const int n = p.Hkv * p.D;
    for (int e = threadIdx.x; e < n; e += 256) {
      const int h = e / p.D;
      const int d = e - h * p.D;
      p.kc[(int64_t)page * p.k_sp + (int64_t)slot * p.k_ss + (int64_t)h * p.k_sh + d] =
          p.nk[(int64_t)b * p.nk_sb + (int64_t)h * p.nk_sh + d];
      p.vc[(int64_t)page * p.v_sp + (int64_t)slot * p.v_ss + (int64_t)h * p.v_sh + d] =
          p.nv[(int64_t)b * p.nv_sb + (int64_t)h * p.nv_sh + d];
    }
  }
  if (advance_here) {
    __syncthreads();
    if (ok && threadIdx.x == 0) p.lens[b] = pos + 1;
  }
}

// One workgroup per sequence, after the scatter: requantise the touched
// (page, head) units of K and V (2 * Hkv units over four waves), then advance
// seq_lens.  Sequences that share a page requantise it with identical results.
template <typename T, int QK, bool VEC>
__global__ __launch_bounds__(256) void append_requant_kernel(const AppendParams p) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int pos, page, slot;
  const bool ok = append_target(p, b, pos, page, slot);
  if (ok) {
    for (int u = wave; u < 2 * p.Hkv; u += 4) {
      const bool is_v = u >= p.Hkv;
      const int h = is_v ? u - p.Hkv : u;
      if (!is_v) {
        quantize_unit<T, QK, VEC>(reinterpret_cast<const uint8_t*>(p.kc + (int64_t)page * p.k_sp + (int64_t)h * p.k_sh),
                                 p.k_ss, p.qk + (int64_t)page * p.qk_sp + (int64_t)h * p.qk_sh, p.qk_ss,
                                 p.ks + (int64_t)page * p.sc_sp + (int64_t)h * p.sc_sh, p.P, p.D, lane);
      } else {
        quantize_unit<T, QK, VEC>(reinterpret_cast<const uint8_t*>(p.vc + (int64_t)page * p.v_sp + (int64_t)h * p.v_sh),
                                 p.v_ss, p.qv + (int64_t)page * p.qv_sp + (int64_t)h * p.qv_sh, p.qv_ss,
                                 p.vs + (int64_t)page * p.sc_sp + (int64_t)h * p.sc_sh, p.P, p.D, lane);
      }
    }
  }
  if (p.advance) {
    __syncthreads();
    if (ok && threadIdx.x == 0) p.lens[b] = pos + 1;
  }
}

}  // namespace fat

// ===========================================================================
// Host side
// ===========================================================================
namespace {

int quant_kind(int32_t dtype) {
  if (dtype == FAT_DTYPE_I8) return fat::Q_I8;
  if (dtype == FAT_DTYPE_FP8E4M3) return fat::Q_FP8;
  return -1;
}

bool aligned(const void* p, int64_t bytes) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0; }

// True when every stride is a multiple of `ch` elements.
bool strides_ok(int64_t ch, std::initializer_list<int64_t> strides) {
  for (int64_t s : strides)
    if (s % ch != 0) return false;
  return true;
}

template <typename S, int QK>
void launch_quant(const fat::QuantParams& prm, bool vec, dim3 grid, hipStream_t stream) {
  if (vec) hipLaunchKernelGGL((fat::quantize_pages_kernel<S, QK, true>), grid, dim3(256), 0, stream, prm);
  else hipLaunchKernelGGL((fat::quantize_pages_kernel<S, QK, false>), grid, dim3(256), 0, stream, prm);
}

template <typename S>
void launch_quant_s(const fat::QuantParams& prm, int qk, bool vec, dim3 grid, hipStream_t stream) {
  if (qk == fat::Q_I8) launch_quant<S, fat::Q_I8>(prm, vec, grid, stream);
  else launch_quant<S, fat::Q_FP8>(prm, vec, grid, stream);
}

template <typename T, int QK>
void launch_requant(const fat::AppendParams& prm, bool vec, dim3 grid, hipStream_t stream) {
  if (vec) hipLaunchKernelGGL((fat::append_requant_kernel<T, QK, true>), grid, dim3(256), 0, stream, prm);
  else hipLaunchKernelGGL((fat::append_requant_kernel<T, QK, false>), grid, dim3(256), 0, stream, prm);
}

template <typename T>
void launch_requant_t(const fat::AppendParams& prm, int qk, bool vec, dim3 grid, hipStream_t stream) {
  if (qk == fat::Q_I8) launch_requant<T, fat::Q_I8>(prm, vec, grid, stream);
  else launch_requant<T, fat::Q_FP8>(prm, vec, grid, stream);
}

}  // namespace

extern "C" int fat_quantize_pages(const fat_quantize_args* a, void* stream_ptr) {
  fat_host::clear_error();
  if (!a || !a->src || !a->dst || !a->scale) {
    fat_host::set_error("fat_quantize_pages: src, dst and scale are required");
    return FAT_E_INVALID;
  }
  if (a->num_pages < 0 || a->page_size <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0) {
    fat_host::set_error("fat_quantize_pages: page_size, num_kv_heads and head_dim must be positive");
    return FAT_E_INVALID;
  }
  const int qk = quant_kind(a->dst_dtype);
  if (qk < 0) {
    fat_host::set_error("fat_quantize_pages: dst_dtype must be int8 or fp8e4m3");
    return FAT_E_UNSUPPORTED;
  }
  int es;
  if (a->src_dtype == FAT_DTYPE_F16 || a->src_dtype == FAT_DTYPE_BF16) es = 2;
  else if (a->src_dtype == FAT_DTYPE_F32) es = 4;
  else {
    fat_host::set_error("fat_quantize_pages: src_dtype must be fp16, bf16 or fp32");
    return FAT_E_UNSUPPORTED;
  }
  const int64_t units = (int64_t)a->num_pages * a->num_kv_heads;
  if (units == 0) return FAT_OK;
  if ((units + 3) / 4 > 0x7fffffffLL) {
    fat_host::set_error("fat_quantize_pages: %lld (page, head) units exceed one launch", (long long)units);
    return FAT_E_UNSUPPORTED;
  }
  fat::QuantParams prm{};
  prm.src = static_cast<const uint8_t*>(a->src);
  prm.dst = static_cast<uint8_t*>(a->dst);
  prm.scale = a->scale;
  prm.s_sp = a->src_stride_page;
  prm.s_ss = a->src_stride_slot;
  prm.s_sh = a->src_stride_head;
  prm.d_sp = a->dst_stride_page;
  prm.d_ss = a->dst_stride_slot;
  prm.d_sh = a->dst_stride_head;
  prm.c_sp = a->scale_stride_page;
  prm.c_sh = a->scale_stride_head;
  prm.num_pages = a->num_pages;
  prm.P = a->page_size;
  prm.Hkv = a->num_kv_heads;
  prm.D = a->head_dim;
  const int64_t ch = 16 / es;
  const bool vec = a->head_dim % ch == 0 && aligned(a->src, 16) && aligned(a->dst, ch) &&
                   strides_ok(ch, {prm.s_sp, prm.s_ss, prm.s_sh, prm.d_sp, prm.d_ss, prm.d_sh});
  const dim3 grid((unsigned)((units + 3) / 4));
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  if (a->src_dtype == FAT_DTYPE_F16) launch_quant_s<fat::F16>(prm, qk, vec, grid, stream);
  else if (a->src_dtype == FAT_DTYPE_BF16) launch_quant_s<fat::BF16>(prm, qk, vec, grid, stream);
  else launch_quant_s<fat::F32>(prm, qk, vec, grid, stream);
  return fat_host::launch_status("quantize_pages_kernel");
}

extern "C" int fat_append_kv(const fat_append_args* a, void* stream_ptr) {
  fat_host::clear_error();
  if (!a || !a->new_k || !a->new_v || !a->k_cache || !a->v_cache || !a->page_table || !a->seq_lens) {
    fat_host::set_error("fat_append_kv: new_k, new_v, k_cache, v_cache, page_table and seq_lens are required");
    return FAT_E_INVALID;
  }
  if (a->batch < 0 || a->num_kv_heads <= 0 || a->head_dim <= 0 || a->page_size <= 0 || a->num_pages <= 0 ||
      a->max_pages <= 0) {
    fat_host::set_error("fat_append_kv: batch must be >= 0 and every other size positive");
    return FAT_E_INVALID;
  }
  if ((int64_t)a->max_pages * a->page_size > 0x7fffffffLL) {
    fat_host::set_error("fat_append_kv: max_pages * page_size overflows int32 positions");
    return FAT_E_INVALID;
  }
  if (a->dtype != FAT_DTYPE_F16 && a->dtype != FAT_DTYPE_BF16) {
    fat_host::set_error("fat_append_kv: the cache dtype must be fp16 or bf16");
    return FAT_E_UNSUPPORTED;
  }
  const bool mirror = a->quant_k_cache || a->quant_v_cache;
  int qk = -1;
  if (mirror) {
    qk = quant_kind(a->quant_dtype);
    if (qk < 0 || !a->quant_k_cache || !a->quant_v_cache || !a->k_scale || !a->v_scale) {
      fat_host::set_error("fat_append_kv: a quantised copy needs int8/fp8 quant_dtype, both code tensors and both "
                          "scale tensors");
      return FAT_E_INVALID;
    }
  }
  if (a->batch == 0) return FAT_OK;
  fat::AppendParams prm{};
  prm.nk = static_cast<const uint16_t*>(a->new_k);
  prm.nv = static_cast<const uint16_t*>(a->new_v);
  prm.kc = static_cast<uint16_t*>(a->k_cache);
  prm.vc = static_cast<uint16_t*>(a->v_cache);
  prm.qk = static_cast<uint8_t*>(a->quant_k_cache);
  prm.qv = static_cast<uint8_t*>(a->quant_v_cache);
  prm.ks = a->k_scale;
  prm.vs = a->v_scale;
  prm.pt = a->page_table;
  prm.lens = a->seq_lens;
  prm.nk_sb = a->new_k_stride_b;
  prm.nk_sh = a->new_k_stride_h;
  prm.nv_sb = a->new_v_stride_b;
  prm.nv_sh = a->new_v_stride_h;
  prm.k_sp = a->k_stride_page;
  prm.k_ss = a->k_stride_slot;
  prm.k_sh = a->k_stride_head;
  prm.v_sp = a->v_stride_page;
  prm.v_ss = a->v_stride_slot;
  prm.v_sh = a->v_stride_head;
  prm.qk_sp = a->qk_stride_page;
  prm.qk_ss = a->qk_stride_slot;
  prm.qk_sh = a->qk_stride_head;
  prm.qv_sp = a->qv_stride_page;
  prm.qv_ss = a->qv_stride_slot;
  prm.qv_sh = a->qv_stride_head;
  prm.sc_sp = a->scale_stride_page;
  prm.sc_sh = a->scale_stride_head;
  prm.pt_sb = a->page_table_stride;
  prm.batch = a->batch;
  prm.Hkv = a->num_kv_heads;
  prm.D = a->head_dim;
  prm.P = a->page_size;
  prm.num_pages = a->num_pages;
  prm.max_pages = a->max_pages;
  prm.advance = a->advance ? 1 : 0;
  const dim3 grid((unsigned)a->batch);
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  hipLaunchKernelGGL(fat::append_scatter_kernel, grid, dim3(256), 0, stream, prm,
                     (!mirror && prm.advance) ? 1 : 0);
  int rc = fat_host::launch_status("append_scatter_kernel");
  if (rc != FAT_OK || !mirror) return rc;
  const bool vec = a->head_dim % 8 == 0 && aligned(a->k_cache, 16) && aligned(a->v_cache, 16) &&
                   aligned(a->quant_k_cache, 8) && aligned(a->quant_v_cache, 8) &&
                   strides_ok(8, {prm.k_sp, prm.k_ss, prm.k_sh, prm.v_sp, prm.v_ss, prm.v_sh, prm.qk_sp, prm.qk_ss,
                                  prm.qk_sh, prm.qv_sp, prm.qv_ss, prm.qv_sh});
  if (a->dtype == FAT_DTYPE_F16) launch_requant_t<fat::F16>(prm, qk, vec, grid, stream);
  else launch_requant_t<fat::BF16>(prm, qk, vec, grid, stream);
  return fat_host::launch_status("append_requant_kernel");
}
