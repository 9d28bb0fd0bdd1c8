// fat_common.h -- device helpers shared by the gfx950 attention kernels.
//
// Everything here is written for CDNA4 wave64: DPP row operations act on
// 16-lane rows, v_permlane{16,32}_swap exchange rows and wave halves, and the
// float conversions map onto single gfx950 instructions (v_cvt_pk_f16_f32,
// v_cvt_pk_bf16_f32, v_cvt_pk_f32_fp8).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/fat_abi.h"

namespace fat {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
// Dword 3 of a raw (stride 0, offset-enabled) gfx950 buffer descriptor.
constexpr int kBufFlags = 0x00020000;

// ---------------------------------------------------------------------------
// Bit casts and 16-bit float pairs packed in one dword.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float as_f32(u32 x) { return __builtin_bit_cast(float, x); }
__device__ __forceinline__ u32 as_u32(float x) { return __builtin_bit_cast(u32, x); }

// Element types as template tags.
struct F16 {};
struct BF16 {};
struct F32 {};

// Element bytes and the final store of one output element of type T.
template <typename T> struct Elem {
  static constexpr int kBytes = 2;
};
template <> struct Elem<F32> {
  static constexpr int kBytes = 4;
};

template <typename T> struct Pair;
template <> struct Pair<F16> {
  static __device__ __forceinline__ float lo(u32 w) { return (float)__builtin_bit_cast(f16x2, w)[0]; }
  static __device__ __forceinline__ float hi(u32 w) { return (float)__builtin_bit_cast(f16x2, w)[1]; }
  // Round two floats to the element type (round to nearest even) and pack.
  static __device__ __forceinline__ u32 pack(float a, float b) {
    f16x2 v = {(f16)a, (f16)b};
    return __builtin_bit_cast(u32, v);
  }
  static __device__ __forceinline__ float dot2(u32 a, u32 b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (f16)x);
  }
};
template <> struct Pair<BF16> {
  static __device__ __forceinline__ float lo(u32 w) { return as_f32(w << 16); }
  static __device__ __forceinline__ float hi(u32 w) { return as_f32(w & 0xffff0000u); }
  static __device__ __forceinline__ u32 pack(float a, float b) {
    bf16x2 v = {(bf16)a, (bf16)b};
    return __builtin_bit_cast(u32, v);
  }
  static __device__ __forceinline__ float dot2(u32 a, u32 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                           false);
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, (bf16)x);
  }
};

// Store x as element `idx` of an output array of element type T (16-bit
// types round to nearest even).
template <typename T>
__device__ __forceinline__ void store_elem(uint8_t* base, int64_t idx, float x) {
  if constexpr (std::is_same<T, F32>::value) {
    reinterpret_cast<float*>(base)[idx] = x;
  } else {
    reinterpret_cast<uint16_t*>(base)[idx] = Pair<T>::from_float(x);
  }
}

// ---------------------------------------------------------------------------
// 8-bit KV storage decoding.  Each returns four floats from one dword.
// ---------------------------------------------------------------------------
// int8: v_cvt_f32_ubyte{0..3} on (w ^ 0x80808080) yields x + 128 exactly;
// the caller folds the -128 into an fma with the scale.
__device__ __forceinline__ void i8x4_biased(u32 w, float* f) {
  u32 u = w ^ 0x80808080u;
  f[0] = (float)(u & 0xffu);
  f[1] = (float)((u >> 8) & 0xffu);
  f[2] = (float)((u >> 16) & 0xffu);
  f[3] = (float)(u >> 24);
}
// OCP e4m3fn (gfx950 converts the OCP encoding natively).
__device__ __forceinline__ void fp8x4(u32 w, float* f) {
  auto a = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  auto b = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  f[0] = a[0];
  f[1] = a[1];
  f[2] = b[0];
  f[3] = b[1];
}

// ---------------------------------------------------------------------------
// Cross-lane primitives.
// ---------------------------------------------------------------------------
// DPP controls (gfx9 encoding).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within each 16 lanes
constexpr int kDppRor4 = 0x124;       // row_ror:4
constexpr int kDppRor8 = 0x128;       // row_ror:8 (== xor 8 inside a row)

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return as_f32((u32)__builtin_amdgcn_mov_dpp((int)as_u32(x), CTRL, 0xF, 0xF, true));
}

// Partner exchange inside a row of LPR lanes that splits on lane bit `BIT`
// and keeps the lane bits above BIT.  Used by the transposing reduction.
template <int BIT>
__device__ __forceinline__ float row_partner(float x) {
  if constexpr (BIT == 8) return dpp<kDppMirror>(x);
  else if constexpr (BIT == 4) return dpp<kDppHalfMirror>(x);
  else if constexpr (BIT == 2) return dpp<kDppXor2>(x);
  else {
    static_assert(BIT == 1, "row_partner: bit must be 1, 2, 4 or 8");
    return dpp<kDppXor1>(x);
  }
}

// Reduction helpers: op(x, partner(x)) over lane-xor masks.
struct OpMax {
  static __device__ __forceinline__ float f(float a, float b) { return fmaxf(a, b); }
};
struct OpAdd {
  static __device__ __forceinline__ float f(float a, float b) { return a + b; }
};

// Combine each lane with lane^16 (both directions in one v_permlane16_swap).
template <typename Op>
__device__ __forceinline__ float xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
  return Op::f(as_f32(r[0]), as_f32(r[1]));
}
// Combine each lane with lane^32.
template <typename Op>
__device__ __forceinline__ float xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
  return Op::f(as_f32(r[0]), as_f32(r[1]));
}

// Reduce over the "row" lane bits of a wave whose lane id is r * LPR + c:
// combines the RPL = 64 / LPR lanes that share c.
template <typename Op, int LPR>
__device__ __forceinline__ float across_rows(float x) {
  static_assert(LPR == 4 || LPR == 8 || LPR == 16, "LPR must be 4, 8 or 16");
  if constexpr (LPR == 4) {
    x = Op::f(x, dpp<kDppRor4>(x));
    x = Op::f(x, dpp<kDppRor8>(x));
  } else if constexpr (LPR == 8) {
    x = Op::f(x, dpp<kDppRor8>(x));
  }
  x = xor16<Op>(x);
  x = xor32<Op>(x);
  return x;
}

// Reduce within a row over the lanes that share the bits above log2(N):
// combines N consecutive lanes (N in {1, 2, 4}).
template <typename Op, int N>
__device__ __forceinline__ float within_quad(float x) {
  static_assert(N == 1 || N == 2 || N == 4, "within_quad: N must be 1, 2 or 4");
  if constexpr (N >= 2) x = Op::f(x, dpp<kDppXor1>(x));
  if constexpr (N >= 4) x = Op::f(x, dpp<kDppXor2>(x));
  return x;
}

// Wave-local LDS ordering: makes this wave's earlier LDS writes visible to its
// later LDS reads (all lanes), without a workgroup barrier.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// Matrix-core helpers shared by the prefill and the MFMA decode.
// ---------------------------------------------------------------------------
template <typename T> struct Mfma;
template <> struct Mfma<F16> {
  static __device__ __forceinline__ f32x16 mma(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
};
template <> struct Mfma<BF16> {
  static __device__ __forceinline__ f32x16 mma(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Transposed 64-bit LDS read: inside each 16-lane group, lane l receives
// element (l % 4) of the 4-element row addressed by lane 4c + l/4, for
// c = 0..3 (gfx950 ds_read_b64_tr_b16).
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}


}  // namespace fat

// ---------------------------------------------------------------------------
// Host side: thread-local error message for fat_last_error().
// ---------------------------------------------------------------------------
namespace fat_host {
void set_error(const char* fmt, ...);
void clear_error();
int launch_status(const char* what);
}  // namespace fat_host
