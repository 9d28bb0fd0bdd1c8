// decode.hip -- single-query paged decode for gfx950 (fp16/bf16/int8/fp8 K/V).
//
// Behaviour follows the FlashAttnTile decode path:
//   flashattn_tile/kernels/decode.py:47-127   (_decode_paged_kernel)
//   flashattn_tile/kernels/decode.py:223-356  (split kernel + LSE reduce)
//   flashattn_tile/kernels/decode.py:359-447  (quantised K/V)
// Design (MI355X-first, not a translation of the Triton programs):
//   * one workgroup per (split, GQA head group, sequence); the HG query heads
//     of a group share one KV head, so every K/V page is read from HBM once
//     per group instead of once per query head;
//   * a wave streams 16-token units (32 at fp16/bf16 head_dim 64); lane
//     (r, c) owns row r of each 16-byte wide load and dims
//     [c*EPL, c*EPL+EPL); K and V rows arrive as global_load_dwordx4, one
//     unit ahead of the compute (register double buffer);
//   * q.k partial sums are reduced across the LPR lanes of a row with a
//     transposing DPP butterfly that leaves one (head, token) score per lane;
//   * softmax state (running max m, sum l) is shared by the whole wave; the
//     probabilities are broadcast to the PV lanes through a few bytes of LDS;
//   * PV accumulates in fp32 (no rounding of p), matching the fp32 oracle;
//   * int8/fp8 pages are dequantised in registers as
//     round_to_q_dtype(float(x) * scale), the reference's own
//     dequantise-then-attend semantics (flashattn_tile/quant.py:145-161);
//     with fp16 queries K is staged exact and k_scale multiplies the fp32
//     scores (the reference's quantised kernel, kernels/decode.py:419-429),
//     and the MFMA decode forms int8 V as x * fp16(scale) (k8_exact_f16);
//   * with split_k > 1 each workgroup writes (acc, m, l) for its partition
//     and a second kernel merges the partitions by log-sum-exp;
//   * multi-token decode (q_len = T > 1, e.g. speculative verification) runs
//     on the MFMA kernel: its 32 MFMA columns are (query head, token) rows,
//     G * T of them per KV head, so each K/V page is still read once per KV
//     head per 32 rows; token t sees keys j <= seq_len - T + t (the
//     bottom-right causal convention of flashattn_tile/reference.py:19-22).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "decode_params.h"

namespace fat {


// Lazy rescale bound of both decode kernels (log2 units): m only moves when
// a block's or unit's max exceeds it by more than this; p then stays below
// 2^kDecLazy.
constexpr float kDecLazy = 8.0f;

// fp16/bf16 K/V with at least this many query heads per KV head use the MFMA
// decode (the `kernel` argument field overrides the choice).
constexpr int kDecMfmaMinGroup = 8;

// K/V rows are read once per launch: streaming (nontemporal) loads.
#ifndef FAT_DEC_NT
#define FAT_DEC_NT 1
#endif
// 16 bytes of K or V at base + off through a raw buffer descriptor of range
// `bytes` (offsets at or past it read as zeros); base is wave-uniform (a
// page's row), off the lane's chunk.  Cache policy 2 is the nt (streaming)
// bit of gfx950 loads.
__device__ __forceinline__ u32x4 kv_buffer_load(const uint8_t* base, int bytes, uint32_t off) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, bytes, kBufFlags);
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, FAT_DEC_NT ? 2 : 0));
}
#ifndef FAT_DEC_MFMA_8BIT
#define FAT_DEC_MFMA_8BIT 1
#endif


// Lane geometry for one 16-byte load per lane.
template <int KV, int D>
struct Geom {
  static constexpr int kElemBytes = (KV == KV_SAME) ? 2 : 1;
  static constexpr int kEpl = 16 / kElemBytes;  // elements per lane per row
  static constexpr int kLpr = D / kEpl;         // lanes per row
  static constexpr int kRpl = 64 / kLpr;        // rows per load
  static constexpr int kNi16 = 16 / kRpl;       // loads per 16 tokens
  // Tokens per streamed unit: 16, or 32 when 16 tokens take only two loads
  // per lane for each of K and V (fp16/bf16 at head_dim 64), so a wave keeps
  // as many bytes in flight as at head_dim 128.
  static constexpr int kUnit = (KV == KV_SAME && kNi16 == 2) ? 32 : 16;
  static constexpr int kUnitLog2 = kUnit == 32 ? 5 : 4;
  static constexpr int kNi = kUnit / kRpl;      // loads per unit
  static_assert(kLpr == 4 || kLpr == 8 || kLpr == 16, "unsupported head_dim / element size");
};

// One transposing butterfly step on lane bit BIT: NCUR values -> NCUR/2.
template <int BIT, int NCUR>
__device__ __forceinline__ void tr_step(float* x, bool up) {
#pragma unroll
  for (int j = 0; j < NCUR / 2; ++j) {
    const float lo = x[j];
    const float hi = x[j + NCUR / 2];
    const float slo = lo + row_partner<BIT>(lo);
    const float shi = hi + row_partner<BIT>(hi);
    x[j] = up ? shi : slo;
  }
}

// Sum N per-lane partials over the LPR lanes of a row; afterwards lane c
// holds the full sums of values j = c * (N / LPR) + k, k < N / LPR.
template <int LPR, int N>
__device__ __forceinline__ void transpose_reduce(float* x, int c) {
  static_assert(N >= LPR, "need at least one value per lane");
  if constexpr (LPR >= 16) tr_step<8, N>(x, (c & 8) != 0);
  if constexpr (LPR >= 8) tr_step<4, N * 8 / LPR>(x, (c & 4) != 0);
  if constexpr (LPR >= 4) tr_step<2, N * 4 / LPR>(x, (c & 2) != 0);
  tr_step<1, N * 2 / LPR>(x, (c & 1) != 0);
}

// Registers holding one unit's K/V rows (and per-load scales for 8-bit K/V).
template <int NI>
struct UnitRegs {
  u32x4 k[NI];
  u32x4 v[NI];
  float ksc[NI];
  float vsc[NI];
};

// 16 bytes of int8 or OCP e4m3 K as their exact values in fp16 (8 packed
// pairs).  With fp16 queries both decode kernels stage K this way and apply
// k_scale to the fp32 scores, as the reference's quantised kernel does
// (kernels/decode.py:419-429: k = float(x) * k_scale, scores in fp32):
// 5 (int8) or 2 (fp8) instructions per 4 elements instead of 11 or 8 for
// round_to_fp16(float(x) * scale).  V keeps that per-element dequantisation:
// folding v_scale into P would round P after a scale that differs per page,
// and pages whose scales differ by 2^15 or more (two can share a 32-key
// block) would leave the smaller one's P in fp16's subnormal range.
template <int KV>
__device__ __forceinline__ void k8_exact_f16(const u32x4& raw, u32 (&out)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (KV == KV_I8) {
      // fp16 bits 0x6400 | u are 1024 + u exactly (u = x + 128, the byte with
      // its sign bit flipped); adding -1152 leaves x.
      const u32 u = raw[j] ^ 0x80808080u;
      const f16x2 bias = {(f16)-1152.0f, (f16)-1152.0f};
      out[2 * j] = __builtin_bit_cast(
          u32, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + bias);
      out[2 * j + 1] = __builtin_bit_cast(
          u32, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + bias);
    } else {  // OCP e4m3 -> fp16 is exact
      out[2 * j] = __builtin_bit_cast(u32, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[j], 1.0f, false));
      out[2 * j + 1] = __builtin_bit_cast(u32, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[j], 1.0f, true));
    }
  }
}

// Page ids of the first unit of keys a wave reads (rows first_row + i * RPL
// of its partition, i < N), loaded at kernel start together with seq_len when
// the partition's first page does not depend on seq_len (partition 0, or
// fixed-size partitions): the first K/V loads then wait one memory latency
// after the launch instead of two.  The indices are clamped into the table
// row.  Two empty asm statements order the loads: the sequence index passes
// through one with the table indices (so the seq_len load issues no earlier
// than the id loads, not ahead of argument loads they wait for), and seq_len
// through one with the ids (so the ids are loaded before seq_len's first use
// instead of where they are used, after the wait for seq_len).  Neither is
// volatile or touches memory, so the loads, and later table reads, stay
// scalar loads.
template <int N, int RPL>
__device__ __forceinline__ int first_page_ids(int* pid, const int32_t* ptrow, const DecodeParams& p, int split,
                                              int first_row, int b, bool early) {
  if (!early) return p.lens[b];
  const int64_t pg0 = p.pps_fixed > 0 ? (int64_t)split * p.pps_fixed : 0;
  int64_t idx[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    idx[i] = min(pg0 + ((first_row + i * RPL) >> p.log2P), (int64_t)p.max_pages - 1);
    asm("" : "+s"(b) : "s"(idx[i]));
  }
  int seq_len = p.lens[b];
#pragma unroll
  for (int i = 0; i < N; ++i) pid[i] = ptrow[idx[i]];
#pragma unroll
  for (int i = 0; i < N; ++i) asm("" : "+s"(pid[i]), "+s"(seq_len));
  return seq_len;
}

// One output element of the split-K merge: row bh (its S partitions'
// (acc, m, l) in the workspace), head dim d, stored at element o of out.
// SMAX (a power of two >= S) fixes the trip count so the loops unroll:
// every partition's (m, l) and acc loads are issued before the first is used,
// one memory latency instead of one per partition.  Padded partitions
// (s >= S) re-read partition S - 1, so every address is inside the row, and
// are then given m = -inf (weight 0).
// COH: the rows were written by other workgroups of this launch with
// device-scope stores (ws_store); they are read with device-scope loads.
template <bool COH>
__device__ __forceinline__ float ws_load(const float* ptr) {
  if constexpr (COH) return __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *ptr;
}
__device__ __forceinline__ void ws_store(float* ptr, float v, bool coh) {
  if (coh) __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *ptr = v;
}

template <typename QT, int SMAX, bool COH = false>
__device__ __forceinline__ void merge_elem(const float* __restrict__ ws_acc, const float* __restrict__ ws_ml,
                                           int64_t bh, int d, int D, int S, uint8_t* out, int64_t o) {
  const float* ml = ws_ml + bh * S * 2;
  const float* acc = ws_acc + bh * S * D + d;
  float m[SMAX], l[SMAX], a[SMAX];
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    const int sc = min(s, S - 1);
    m[s] = ws_load<COH>(ml + 2 * sc);
    l[s] = ws_load<COH>(ml + 2 * sc + 1);
    a[s] = ws_load<COH>(acc + (int64_t)sc * D);
  }
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    if (s >= S) {
      m[s] = -INFINITY;
      l[s] = 0.f;
      a[s] = 0.f;
    }
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < SMAX; ++s) M = fmaxf(M, m[s]);
  float A = 0.f, L = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      const float f = fast_exp2(m[s] - M);  // 0 for padded or empty partitions
      A = __builtin_fmaf(a[s], f, A);
      L = __builtin_fmaf(l[s], f, L);
    }
  }
  store_elem<QT>(out, o, L > 0.f ? A / L : 0.f);
}

// The merge of merge_in_launch, with merge_elem's arithmetic: per row j (one
// thread each) M = max_s m_s, the weights f_s = 2^(m_s - M) (0 for padded
// partitions) and L = sum_s l_s f_s in partition order, kept in LDS; per
// output element A = sum_s acc_s f_s in partition order and A / L.  A
// thread takes at most two elements (the host fuses the merge only then)
// and issues their partial sums' loads together with its row's (m, l), so
// the merge waits for one memory latency.
template <typename QT, int D, int SMAX, typename RowOf>
__device__ __forceinline__ void merge_rows(const DecodeParams& p, int S, int nrows, RowOf row_of, float* s_f,
                                           float* s_l) {
  const int n = nrows * D;
  const int e0 = threadIdx.x, e1 = threadIdx.x + blockDim.x;  // this thread's elements (if < n)
  float a0[SMAX], a1[SMAX];
  int64_t o0 = 0, o1 = 0;
  auto load_acc = [&](int e, float (&a)[SMAX], int64_t& o) {
    const int j = e / D;
    const int d = e - j * D;
    int64_t bh;
    row_of(j, bh, o);
    o += d;
    const float* acc = p.ws_acc + bh * S * D + d;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) a[s] = s < S ? ws_load<true>(acc + (int64_t)s * D) : 0.f;
  };
  if (e0 < n) load_acc(e0, a0, o0);
  if (e1 < n) load_acc(e1, a1, o1);
  if (threadIdx.x < nrows) {
    const int j = threadIdx.x;
    int64_t bh, o;
    row_of(j, bh, o);
    const float* ml = p.ws_ml + bh * S * 2;
    float m[SMAX], l[SMAX];
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      const int sc = min(s, S - 1);
      m[s] = ws_load<true>(ml + 2 * sc);
      l[s] = ws_load<true>(ml + 2 * sc + 1);
    }
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      if (s >= S) {
        m[s] = -INFINITY;
        l[s] = 0.f;
      }
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) M = fmaxf(M, m[s]);
    float L = 0.f;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      const float f = M != -INFINITY ? fast_exp2(m[s] - M) : 0.f;
      s_f[j * SMAX + s] = f;
      L = __builtin_fmaf(l[s], f, L);
    }
    s_l[j] = M != -INFINITY ? L : -1.f;  // -1: no partition saw a key (output 0, as merge_elem)
  }
  __syncthreads();
  auto finish = [&](int e, const float (&a)[SMAX], int64_t o) {
    const int j = e / D;
    const float L = s_l[j];
    float A = 0.f;
    if (L >= 0.f) {
#pragma unroll
      for (int s = 0; s < SMAX; ++s) A = __builtin_fmaf(a[s], s_f[j * SMAX + s], A);
    }
    store_elem<QT>(p.out, o, L > 0.f ? A / L : 0.f);
  };
  if (e0 < n) finish(e0, a0, o0);
  if (e1 < n) finish(e1, a1, o1);
}

// Split-K merge inside the decode launch (p.counters set).  Every thread has
// written its part of this workgroup's (acc, m, l) rows with device-scope
// stores (ws_store, global_store ... sc1: written through to the level all
// XCDs share); each wave waits until its stores have completed there
// (vmcnt(0)), then the workgroup counts itself in on its (sequence, head
// group) counter with a device-scope atomic.  The workgroup that brings the
// count to S has therefore seen every other partition's count, each issued
// after that partition's rows were complete at the shared level; it reads
// them with device-scope loads (global_load ... sc1), merges them and puts
// the counter back to zero for the next launch.  The ordering rests on
// those gfx950 completion rules, not on release/acquire operations: an
// agent-scope release would write back the whole L2 of the XCD
// (buffer_wbl2), which measured 7-16 % slower on 8-sequence split
// launches.  No workgroup waits for another.
template <typename QT, int D, typename RowOf>
__device__ __forceinline__ void merge_in_launch(const DecodeParams& p, int S, int nrows, RowOf row_of) {
  __shared__ int s_last;
  __shared__ float s_f[32 * 16];  // merge weights of up to 32 rows x 16 partitions
  __shared__ float s_l[32];
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // keep the row stores before the wait
  __builtin_amdgcn_s_waitcnt(0x0F70);       // vmcnt(0): this wave's row stores are complete
  __syncthreads();
  int* const cnt = p.counters + (blockIdx.z * gridDim.y + blockIdx.y);
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == S - 1;
  }
  __syncthreads();
  if (!s_last) return;
  switch (p.smax) {
    case 4: merge_rows<QT, D, 4>(p, S, nrows, row_of, s_f, s_l); break;
    case 8: merge_rows<QT, D, 8>(p, S, nrows, row_of, s_f, s_l); break;
    default: merge_rows<QT, D, 16>(p, S, nrows, row_of, s_f, s_l); break;
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename QT, int KV, int D, int HG, int NW>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(const DecodeParams p) {
  using Gm = Geom<KV, D>;
  constexpr int EPL = Gm::kEpl, LPR = Gm::kLpr, RPL = Gm::kRpl, NI = Gm::kNi;
  constexpr int NV = NI * HG;       // per-lane partial scores before the reduction
  constexpr int NPL = NV / LPR;     // scores per lane after it
  constexpr int VPH = NPL < NI ? NPL : NI;  // scores per lane per head
  constexpr int HPL = NPL / VPH;            // heads per lane
  constexpr int LPH = NI / VPH;             // lanes per head inside a row
  constexpr int QW = EPL / 2;               // q dwords per head per lane (packed pairs)
  static_assert(HG % 4 == 0, "HG must be a multiple of 4");

  __shared__ float s_p[NW][RPL][NV];
  __shared__ float s_alpha[NW][HG];
  __shared__ float s_red[NW][HG][D];
  __shared__ float s_ml[NW][HG][2];

  const int split = blockIdx.x;
  const int S = gridDim.x;
  const int y = blockIdx.y;
  const int b = blockIdx.z;
  const int sub = y % p.hg_per_kv;
  const int kvh = y / p.hg_per_kv;
  const int head0 = kvh * p.group + sub * HG;
  const int nvalid = min(HG, p.group - sub * HG);

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane / LPR;
  const int c = lane % LPR;

  // Page ids of this wave's first unit, read together with seq_len when
  // `early` (first_page_ids); rows of that unit past the sequence's end read
  // the table again (fetch).
  constexpr int UL = Gm::kUnitLog2;
  const int32_t* ptrow = p.pt + (int64_t)b * p.pt_sb;
  const bool early = split == 0 || p.pps_fixed > 0;
  int first_pid[NI];
  // Partition of this sequence's pages (decode.py:271-276 semantics).
  int seq_len = first_page_ids<NI, RPL>(first_pid, ptrow, p, split, w << UL, b, early);
  seq_len = max(0, min(seq_len, p.max_pages << p.log2P));
  const int np = (seq_len + p.P - 1) >> p.log2P;
  const int pps = p.pps_fixed > 0 ? p.pps_fixed : (np + S - 1) / S;
  const int pb = split * pps;
  const int pe = split == S - 1 ? np : min(np, pb + pps);
  const int t_begin = pb << p.log2P;
  const int t_end = min(seq_len, pe << p.log2P);
  const int n_units = t_end > t_begin ? (t_end - t_begin + Gm::kUnit - 1) >> UL : 0;

  // q for the HG heads, packed pairs of QT (padded heads reuse head0).
  u32 qv[HG][QW];
#pragma unroll
  for (int g = 0; g < HG; ++g) {
    const int h = head0 + (g < nvalid ? g : 0);
    const u32x4* qp = reinterpret_cast<const u32x4*>(p.q + 2 * (b * p.q_sb + h * p.q_sh + c * EPL));
#pragma unroll
    for (int j = 0; j < QW / 4; ++j) {
      const u32x4 t = qp[j];
      qv[g][4 * j + 0] = t[0];
      qv[g][4 * j + 1] = t[1];
      qv[g][4 * j + 2] = t[2];
      qv[g][4 * j + 3] = t[3];
    }
  }

  constexpr int EB = Gm::kElemBytes;
  // Load i of a unit covers rows rs .. rs + RPL - 1 of one page (page_size
  // >= RPL, rs a multiple of RPL): its address is wave-uniform (page id,
  // slot and KV head on the scalar unit, in a buffer descriptor) plus this
  // lane's loop-invariant offset (row r, chunk c).  The descriptor's range
  // ends with the partition's last row, so rows past t_end (and loads wholly
  // past it) read as zeros: their scores are masked, and zero V rows keep
  // p * v = 0.
  // Byte strides (the host keeps a page below 4 GB and RPL rows below 2 GB).
  const uint8_t* const kh = p.k + (int64_t)EB * kvh * p.k_sh;  // this KV head's slice of page 0
  const uint8_t* const vh = p.v + (int64_t)EB * kvh * p.v_sh;
  const uint32_t kpage = (uint32_t)(EB * p.k_sp), vpage = (uint32_t)(EB * p.v_sp);
  const uint32_t krow = (uint32_t)(EB * p.k_ss), vrow = (uint32_t)(EB * p.v_ss);
  const uint32_t lane_k = r * krow + EB * EPL * c;
  const uint32_t lane_v = r * vrow + EB * EPL * c;

  // first: u is this wave's first unit (first_pid holds its page ids).
  auto fetch = [&](UnitRegs<NI>& R, int u, bool first) {
    const int base = t_begin + (u << UL);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int rs = base + i * RPL;
      const int nrow = min(t_end - rs, RPL);  // rows of this load in the partition
      // The table is read without a branch (at most its last entry) so that
      // a unit's page-id loads issue together; a load wholly past t_end reads
      // nothing (range 0).
      int phys = first && early ? first_pid[i] : ptrow[min(rs >> p.log2P, p.max_pages - 1)];
      phys = __builtin_amdgcn_readfirstlane(min(max(phys, 0), p.num_pages - 1));
      const uint32_t slot0 = (uint32_t)(rs & (p.P - 1));
      // range: the load's rows inside the partition, each up to its head slice's end
      const int nk = nrow > 0 ? (int)((uint32_t)(nrow - 1) * krow + EB * D) : 0;
      const int nv = nrow > 0 ? (int)((uint32_t)(nrow - 1) * vrow + EB * D) : 0;
      R.k[i] = kv_buffer_load(kh + (uint64_t)(uint32_t)phys * kpage + slot0 * krow, nk, lane_k);
      R.v[i] = kv_buffer_load(vh + (uint64_t)(uint32_t)phys * vpage + slot0 * vrow, nv, lane_v);
      if constexpr (KV != KV_SAME) {
        R.ksc[i] = p.ks[(int64_t)phys * p.sc_sp + (int64_t)kvh * p.sc_sh];
        R.vsc[i] = p.vs[(int64_t)phys * p.sc_sp + (int64_t)kvh * p.sc_sh];
      }
    }
  };

  // FOLD: exact 8-bit K and k_scale on the scores (k8_exact_f16).
  constexpr bool FOLD = KV != KV_SAME && std::is_same<QT, F16>::value;
  // Dequantise 16 bytes of 8-bit K/V into EPL/2 packed QT pairs:
  // round_to_QT(float(x) * scale).
  auto deq_pairs = [&](const u32x4& raw, float sc, u32* out) {
    const float nb = -128.0f * sc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float f[4];
      if constexpr (KV == KV_I8) {
        i8x4_biased(raw[j], f);
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = __builtin_fmaf(f[e], sc, nb);
      } else {
        fp8x4(raw[j], f);
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = f[e] * sc;
      }
      out[2 * j + 0] = Pair<QT>::pack(f[0], f[1]);
      out[2 * j + 1] = Pair<QT>::pack(f[2], f[3]);
    }
  };

  float m_run[HPL], l_run[HPL];
#pragma unroll
  for (int hh = 0; hh < HPL; ++hh) {
    m_run[hh] = -INFINITY;
    l_run[hh] = 0.f;
  }
  float acc[HG][EPL];
#pragma unroll
  for (int g = 0; g < HG; ++g)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;

  // One unit: scores, online softmax, PV.
  auto process = [&](const UnitRegs<NI>& cur, int u) __attribute__((always_inline)) {
    const int base = t_begin + (u << UL);

    // ---- scores: partial q.k over this lane's EPL dims ----
    float part[NV];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      u32 kw[QW];
      if constexpr (KV == KV_SAME) {
#pragma unroll
        for (int j = 0; j < 4; ++j) kw[j] = cur.k[i][j];
      } else if constexpr (FOLD) {
        k8_exact_f16<KV>(cur.k[i], kw);
      } else {
        deq_pairs(cur.k[i], cur.ksc[i], kw);
      }
#pragma unroll
      for (int g = 0; g < HG; ++g) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < QW; ++j) s = Pair<QT>::dot2(qv[g][j], kw[j], s);
        part[g * NI + i] = FOLD ? s * cur.ksc[i] : s;  // load i's rows share one page
      }
    }
    transpose_reduce<LPR, NV>(part, c);

    // ---- online softmax (state shared by the wave, per head) ----
    float pr[NPL];
    float alpha[HPL];
#pragma unroll
    for (int hh = 0; hh < HPL; ++hh) {
      float mx = -INFINITY;
#pragma unroll
      for (int v = 0; v < VPH; ++v) {
        const int k = hh * VPH + v;
        const int j = c * NPL + k;
        const int i = j % NI;
        const bool valid = base + i * RPL + r < t_end;
        const float s = valid ? part[k] * p.scale_log2 : -INFINITY;
        pr[k] = s;
        mx = fmaxf(mx, s);
      }
      mx = within_quad<OpMax, LPH>(mx);
      mx = across_rows<OpMax, LPR>(mx);
      // Lazy max: m moves (and acc / l are rescaled) only when a unit's max
      // exceeds it by more than kDecLazy, so p = 2^(s - m) stays below
      // 2^kDecLazy -- exact in the fp32 sums and PV -- and most units skip
      // the rescale.
      const bool grow = mx > m_run[hh] + kDecLazy;
      const float m_new = grow ? mx : m_run[hh];
      alpha[hh] = grow ? fast_exp2(m_run[hh] - m_new) : 1.f;
      float ps = 0.f;
#pragma unroll
      for (int v = 0; v < VPH; ++v) {
        const int k = hh * VPH + v;
        pr[k] = fast_exp2(pr[k] - m_new);
        ps += pr[k];
      }
      l_run[hh] = l_run[hh] * alpha[hh] + ps;
      m_run[hh] = m_new;
    }

    // ---- broadcast p (per row) and alpha (per wave) through LDS ----
#pragma unroll
    for (int k = 0; k < NPL; ++k) s_p[w][r][c * NPL + k] = pr[k];
    if (r == 0) {
#pragma unroll
      for (int hh = 0; hh < HPL; ++hh) {
        const int j0 = c * NPL + hh * VPH;
        if (j0 % NI == 0) s_alpha[w][j0 / NI] = alpha[hh];
      }
    }
    wave_lds_fence();
    float pv[NV];
    float al[HG];
#pragma unroll
    for (int j = 0; j < NV; j += 4) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(&s_p[w][r][j]);
      pv[j] = t[0];
      pv[j + 1] = t[1];
      pv[j + 2] = t[2];
      pv[j + 3] = t[3];
    }
#pragma unroll
    for (int g = 0; g < HG; g += 4) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(&s_alpha[w][g]);
      al[g] = t[0];
      al[g + 1] = t[1];
      al[g + 2] = t[2];
      al[g + 3] = t[3];
    }
    wave_lds_fence();

    // ---- acc = acc * alpha + sum_i p_i * v_i (fp32) ----
    // al[] is the same for every lane of the wave (read back from LDS).
    bool rescale = false;
#pragma unroll
    for (int g = 0; g < HG; ++g) rescale |= al[g] != 1.f;
    if (rescale) {
#pragma unroll
      for (int g = 0; g < HG; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] *= al[g];
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float vf[EPL];
      u32 vw[QW];
      if constexpr (KV == KV_SAME) {
#pragma unroll
        for (int j = 0; j < 4; ++j) vw[j] = cur.v[i][j];
      } else {
        deq_pairs(cur.v[i], cur.vsc[i], vw);
      }
#pragma unroll
      for (int j = 0; j < QW; ++j) {
        vf[2 * j] = Pair<QT>::lo(vw[j]);
        vf[2 * j + 1] = Pair<QT>::hi(vw[j]);
      }
#pragma unroll
      for (int g = 0; g < HG; ++g) {
        const float pg = pv[g * NI + i];
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(pg, vf[e], acc[g][e]);
      }
    }
  };

  // Two register sets, unit u + NW loading while unit u is processed (the
  // loop is unrolled by two so that no copy moves one set into the other).
  UnitRegs<NI> nxt;
  if (w < n_units) fetch(nxt, w, true);
  for (int u = w; u < n_units; u += NW) {
    const UnitRegs<NI> cur = nxt;
    if (u + NW < n_units) fetch(nxt, u + NW, false);
    process(cur, u);
  }

  // ---- merge rows of the wave (same m), then the waves of the workgroup ----
#pragma unroll
  for (int hh = 0; hh < HPL; ++hh) {
    float l = within_quad<OpAdd, LPH>(l_run[hh]);
    l_run[hh] = across_rows<OpAdd, LPR>(l);
  }
#pragma unroll
  for (int g = 0; g < HG; ++g)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = across_rows<OpAdd, LPR>(acc[g][e]);
  if (r == 0) {
#pragma unroll
    for (int g = 0; g < HG; ++g)
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_red[w][g][c * EPL + e] = acc[g][e];
#pragma unroll
    for (int hh = 0; hh < HPL; ++hh) {
      const int j0 = c * NPL + hh * VPH;
      if (j0 % NI == 0) {
        s_ml[w][j0 / NI][0] = m_run[hh];
        s_ml[w][j0 / NI][1] = l_run[hh];
      }
    }
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < HG * D; idx += NW * 64) {
    const int g = idx / D;
    const int d = idx % D;
    if (g >= nvalid) continue;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, s_ml[ww][g][0]);
    float A = 0.f, L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float f = fast_exp2(s_ml[ww][g][0] - M);
        A = __builtin_fmaf(s_red[ww][g][d], f, A);
        L = __builtin_fmaf(s_ml[ww][g][1], f, L);
      }
    }
    const int h = head0 + g;
    if (S == 1) {
      const float o = L > 0.f ? A / L : 0.f;
      uint16_t* op = reinterpret_cast<uint16_t*>(p.out) + (b * p.o_sb + h * p.o_sh + d);
      *op = Pair<QT>::from_float(o);
    } else {
      const int64_t row = ((int64_t)b * p.H + h) * S + split;
      const bool coh = p.counters != nullptr;
      ws_store(p.ws_acc + row * D + d, A, coh);
      if (d == 0) {
        ws_store(p.ws_ml + row * 2 + 0, M, coh);
        ws_store(p.ws_ml + row * 2 + 1, L, coh);
      }
    }
  }
  if (S > 1 && p.counters) {
    merge_in_launch<QT, D>(p, S, nvalid, [&](int j, int64_t& bh, int64_t& o) {
      const int h = head0 + j;
      bh = (int64_t)b * p.H + h;
      o = (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
    });
  }
}

// ---------------------------------------------------------------------------
// MFMA decode for large GQA groups (group >= 8, e.g. MQA 32/1): one workgroup
// per (partition, KV head, up to 32 of its query heads, sequence).  With G
// query heads per KV head every K/V byte feeds 2G FLOPs, more than the VALU
// sustains at HBM speed for G >= 8, so both products run on the matrix core:
//   S^T = K Q^T   v_mfma_f32_32x32x16: A = 32 keys x 16 dims straight from
//                 each lane's own 16-byte K loads (the head dims are permuted
//                 identically in K and Q so those loads stay contiguous),
//                 B = Q^T of the 32 heads (registers, loaded once);
//   O^T += V^T P^T  A = V^T through the wave's LDS tile (ds_read_b64_tr_b16),
//                 B = P^T straight from the S^T accumulator.
// Each wave streams its own 32-key blocks (wave-private LDS, no workgroup
// barrier in the loop) with its own online softmax; the waves merge at the
// end, and partitions go through the same log-sum-exp merge as the VALU
// kernel.  P is rounded to the K/V type for PV (bf16: hi + lo parts).
// ---------------------------------------------------------------------------
// NW = 4 or 8 waves per workgroup: the host takes 8 when the grid has fewer
// than two workgroups per CU, so each CU still streams 8 blocks at a time.
template <typename QT, int KV, int D, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void paged_decode_mfma_kernel(const DecodeParams p) {
  constexpr int KS = D / 16;     // MFMA k-steps
  constexpr int DB = D / 32;     // 32-dim blocks of O^T
  constexpr int K_RS = D + 8;    // LDS row strides (elements) of the K and V
  constexpr int V_RS = D + 32;   // tiles, spreading reads over the banks
  constexpr bool SPLIT_P = std::is_same<QT, BF16>::value;
  constexpr int EB = KV == KV_SAME ? 2 : 1;        // bytes per stored element
  // Row-coalesced loads: CPR lanes cover one stored row with 16-byte chunks
  // (EPC elements each); one load instruction covers RPL rows, so a 32-key
  // block takes NLD loads per lane for K and as many for V.
  constexpr int EPC = 16 / EB;
  constexpr int CPR = D / EPC;
  constexpr int RPL = 64 / CPR;
  constexpr int NLD = 32 / RPL;
  static_assert(CPR * EPC == D && NLD * RPL == 32, "unsupported head_dim / element size");

  // K and V tiles during the loop; per-wave O / m / l for the merge after it.
  constexpr int kTileBytes = NW * 32 * (K_RS + V_RS) * 2;
  constexpr int kMergeBytes = (NW * 32 * D + NW * 32 * 2) * 4;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kTileBytes > kMergeBytes ? kTileBytes : kMergeBytes];

  const int split = blockIdx.x;
  const int S = gridDim.x;
  const int y = blockIdx.y;
  const int b = blockIdx.z;
  const int sub = y % p.hg_per_kv;
  const int kvh = y / p.hg_per_kv;
  // The workgroup's 32 columns are rows r = sub * 32 + c of this KV head's
  // group * T (query head, token) pairs: head kvh * group + r % group, token
  // r / group (T = 1: the heads of the group).
  const int row_base = sub * 32;
  const int nvalid = min(32, p.group * p.T - row_base);

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31;  // key row (A operand) / (head, token) column (B, S^T)
  const int g = lane >> 5;   // k-group: head dims 16ks + 8g .. +7 of k-step ks

  // Page ids of this wave's first 32-key block, read together with seq_len
  // when `early` (first_page_ids).
  const int32_t* ptrow = p.pt + (int64_t)b * p.pt_sb;
  const bool early = split == 0 || p.pps_fixed > 0;
  int first_pid[NLD];
  int seq_len = first_page_ids<NLD, RPL>(first_pid, ptrow, p, split, w << 5, b, early);
  seq_len = max(0, min(seq_len, p.max_pages << p.log2P));
  const int np = (seq_len + p.P - 1) >> p.log2P;
  const int pps = p.pps_fixed > 0 ? p.pps_fixed : (np + S - 1) / S;
  const int pb = split * pps;
  const int pe = split == S - 1 ? np : min(np, pb + pps);
  const int t_begin = pb << p.log2P;
  const int t_end = min(seq_len, pe << p.log2P);
  const int n_blocks = t_end > t_begin ? (t_end - t_begin + 31) >> 5 : 0;
  // This lane's column: (query head, token) and the end of its visible keys.
  const int my_r = row_base + min(li, nvalid - 1);
  const int my_t = my_r / p.group;
  const int my_h = kvh * p.group + (my_r - my_t * p.group);
  const int my_end = min(t_end, seq_len - p.T + 1 + my_t);

  // Q^T: lane (column li, k-group g), k-step ks = head dims 16ks + 8g + 0..7.
  u32x4 qf[KS];
  {
    const uint8_t* qp = p.q + 2 * ((int64_t)b * p.q_sb + (int64_t)my_t * p.q_st + (int64_t)my_h * p.q_sh + 8 * g);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const u32x4*>(qp + 32 * ks);
  }

  const int lrow = lane / CPR;  // this lane's row inside each load
  const int lcol = lane % CPR;  // and its 16-byte chunk
  // Raw K/V chunks of a 32-key block: load i covers rows RPL*i .. RPL*i +
  // RPL - 1, which lie in one page (page_size >= RPL), so its page id and
  // (8-bit caches) scales are wave-uniform.  Its address is that page's
  // base (scalar unit, in a buffer descriptor) plus this lane's
  // loop-invariant offset; the descriptor's range ends with the partition's
  // last row, so rows past t_end read as zeros (their scores are masked, and
  // zero bytes are zero in every cache type).
  const uint8_t* const kh = p.k + (int64_t)EB * kvh * p.k_sh;  // this KV head's slice of page 0
  const uint8_t* const vh = p.v + (int64_t)EB * kvh * p.v_sh;
  const uint32_t kpage = (uint32_t)(EB * p.k_sp), vpage = (uint32_t)(EB * p.v_sp);
  const uint32_t krow = (uint32_t)(EB * p.k_ss), vrow = (uint32_t)(EB * p.v_ss);
  const uint32_t lane_k = lrow * krow + 16 * lcol;
  const uint32_t lane_v = lrow * vrow + 16 * lcol;
  struct Raw {
    u32x4 k[NLD], v[NLD];
    float ksc[NLD], vsc[NLD];
  };
  // first: blk is this wave's first block (first_pid holds its page ids).
  auto fetch = [&](Raw& R, int blk, bool first) {
    const int kb = t_begin + (blk << 5);
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int rs = kb + i * RPL;
      const int nrow = min(t_end - rs, RPL);  // rows of this load in the partition
      // read without a branch (at most the table's last entry); a load wholly
      // past t_end reads nothing (range 0)
      int phys = first && early ? first_pid[i] : ptrow[min(rs >> p.log2P, p.max_pages - 1)];
      phys = __builtin_amdgcn_readfirstlane(min(max(phys, 0), p.num_pages - 1));
      const uint32_t slot0 = (uint32_t)(rs & (p.P - 1));
      const int nk = nrow > 0 ? (int)((uint32_t)(nrow - 1) * krow + EB * D) : 0;
      const int nv = nrow > 0 ? (int)((uint32_t)(nrow - 1) * vrow + EB * D) : 0;
      R.k[i] = kv_buffer_load(kh + (uint64_t)(uint32_t)phys * kpage + slot0 * krow, nk, lane_k);
      R.v[i] = kv_buffer_load(vh + (uint64_t)(uint32_t)phys * vpage + slot0 * vrow, nv, lane_v);
      if constexpr (KV != KV_SAME) {
        R.ksc[i] = p.ks[(int64_t)phys * p.sc_sp + (int64_t)kvh * p.sc_sh];
        R.vsc[i] = p.vs[(int64_t)phys * p.sc_sp + (int64_t)kvh * p.sc_sh];
      }
    }
  };
  // FOLD (8-bit cache, fp16 queries): exact 8-bit K and k_scale on the
  // scores (k8_exact_f16).  int8 V as x * fp16(v_scale), one packed fp16
  // multiply per pair (FOLD_V): within one fp16 ulp of round_to_fp16(
  // float(x) * v_scale) (the scale's own rounding to fp16 is the second
  // rounding; a scale below fp16's normal range, 6.1e-5, can be off by up to
  // 3e-8, i.e. a V error below 4e-6), inside the dequantise-then-attend
  // tolerance.  fp8 V keeps the fp32 dequantise, which measured faster there.
  constexpr bool FOLD = KV != KV_SAME && std::is_same<QT, F16>::value;
  constexpr bool FOLD_V = FOLD && KV == KV_I8;
  // Store one raw chunk as QT elements at dst (EPC of them): a copy for
  // fp16/bf16 caches, round_to_QT(float(x) * scale) for 8-bit ones, or
  // (put_exact, FOLD K) the exact 8-bit values.
  auto put_exact = [&](uint16_t* dst, const u32x4& raw) {
    u32 o[8];
    k8_exact_f16<KV>(raw, o);
    *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(dst + 8) = u32x4{o[4], o[5], o[6], o[7]};
  };
  auto put_scaled = [&](uint16_t* dst, const u32x4& raw, float sc) {
    u32 o[8];
    k8_exact_f16<KV>(raw, o);
    const f16x2 s2 = {(f16)sc, (f16)sc};
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = __builtin_bit_cast(u32, __builtin_bit_cast(f16x2, o[j]) * s2);
    *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(dst + 8) = u32x4{o[4], o[5], o[6], o[7]};
  };
  auto put = [&](uint16_t* dst, const u32x4& raw, float sc) {
    if constexpr (KV == KV_SAME) {
      *reinterpret_cast<u32x4*>(dst) = raw;
    } else {
      const float nb = -128.0f * sc;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float f[4];
          if constexpr (KV == KV_I8) {
            i8x4_biased(raw[2 * h2 + j], f);
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = __builtin_fmaf(f[e], sc, nb);
          } else {
            fp8x4(raw[2 * h2 + j], f);
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = f[e] * sc;
          }
          o[2 * j] = Pair<QT>::pack(f[0], f[1]);
          o[2 * j + 1] = Pair<QT>::pack(f[2], f[3]);
        }
        *reinterpret_cast<u32x4*>(dst + 8 * h2) = o;
      }
    }
  };

  uint16_t* const Kt = reinterpret_cast<uint16_t*>(smem) + w * 32 * (K_RS + V_RS);
  uint16_t* const Vt = Kt + 32 * K_RS;
  const int tr_c = (lane & 15) >> 2;
  const int tr_j = lane & 3;
  const int tr_G = lane >> 4;
  const int tr_row = 4 * (tr_G >> 1) + tr_c;
  const int tr_col = 16 * (tr_G & 1) + 4 * tr_j;

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  float m_run = -INFINITY;  // log2 units
  float l_run = 0.f;
  const float c = p.scale_log2;

  // One 32-key block from R; refills R with block nxt once R is consumed.
  auto compute = [&](Raw& R, int blk, int nxt) {
    // K(blk) and V(blk) into this wave's LDS tiles (row = key, columns =
    // head dims), then R is free for the next block's loads.
    float ck[NLD];  // FOLD: score factor (softmax scale times k_scale) per load
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int row = i * RPL + lrow;
      if constexpr (FOLD) {
        ck[i] = c * R.ksc[i];
        put_exact(&Kt[row * K_RS + lcol * EPC], R.k[i]);
      } else {
        put(&Kt[row * K_RS + lcol * EPC], R.k[i], R.ksc[i]);
      }
      if constexpr (FOLD_V) {
        put_scaled(&Vt[row * V_RS + lcol * EPC], R.v[i], R.vsc[i]);
      } else {
        put(&Vt[row * V_RS + lcol * EPC], R.v[i], R.vsc[i]);
      }
    }
    if (nxt < n_blocks) fetch(R, nxt, false);
    wave_lds_fence();
    // S^T = K Q^T for the 32 keys of this block: A = K rows li, dims 16ks + 8g.
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(&Kt[li * K_RS + 16 * ks + 8 * g]);
      s = Mfma<QT>::mma(a, qf[ks], s);
    }

    // Online softmax for column li over keys kb + (r&3) + 4g + 8(r>>2).
    const int kb = t_begin + (blk << 5);
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + (r & 3) + 4 * g + 8 * (r >> 2);
      // key row 8 (r >> 2) + (r & 3) + 4g of the block: load (r >> 2) * 8 / RPL
      const float cr = FOLD ? ck[(r >> 2) * 8 / RPL] : c;
      const float x = key < my_end ? s[r] * cr : -INFINITY;
      s[r] = x;
      mx = fmaxf(mx, x);
    }
    mx = xor32<OpMax>(mx);
    if (__any(mx > m_run + kDecLazy)) {
      const bool grow = mx > m_run + kDecLazy;
      const float alpha = grow ? fast_exp2(m_run - mx) : 1.f;
      m_run = grow ? mx : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
    }
    // A column that has seen no visible key yet (only possible for T > 1)
    // keeps m = -inf; its scores are -inf too, and exp2(-inf - 0) = 0.
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    u32x4 pf[2], pl[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const float x0 = fast_exp2(s[8 * t + 2 * e2] - m_use);
        const float x1 = fast_exp2(s[8 * t + 2 * e2 + 1] - m_use);
        l_run += x0 + x1;
        const u32 hp = Pair<QT>::pack(x0, x1);
        pf[t][e2] = hp;
        if constexpr (SPLIT_P) pl[t][e2] = Pair<QT>::pack(x0 - Pair<QT>::lo(hp), x1 - Pair<QT>::hi(hp));
      }
    wave_lds_fence();
    // O^T += V^T P^T (k-step t covers keys 16t..16t+15 of the block).
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int vrow = 16 * t + tr_row;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint16_t* vp = &Vt[vrow * V_RS + 32 * db + tr_col];
        const u32x2 lo = lds_read_tr16(vp);
        const u32x2 hi2 = lds_read_tr16(vp + 8 * V_RS);
        const u32x4 a = {lo[0], lo[1], hi2[0], hi2[1]};
        acc[db] = Mfma<QT>::mma(a, pf[t], acc[db]);
        if constexpr (SPLIT_P) acc[db] = Mfma<QT>::mma(a, pl[t], acc[db]);
      }
    }
    wave_lds_fence();
  };
  Raw R;
  if (w < n_blocks) fetch(R, w, true);
  for (int blk = w; blk < n_blocks; blk += NW) compute(R, blk, blk + NW);

  // ---- merge the waves: O = sum_w acc_w 2^(m_w - M) / sum_w l_w 2^(m_w - M) ----
  __syncthreads();  // every wave is done with its V tile (smem is reused)
  float* so = reinterpret_cast<float*>(smem);   // [NW][32 heads][D]
  float* sml = so + NW * 32 * D;                // [NW][32 heads][2]
  const float l_tot = xor32<OpAdd>(l_run);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) so[(w * 32 + li) * D + 32 * db + (r & 3) + 4 * g + 8 * (r >> 2)] = acc[db][r];
  if (g == 0) {
    sml[(w * 32 + li) * 2 + 0] = m_run;
    sml[(w * 32 + li) * 2 + 1] = l_tot;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < nvalid * D; idx += NW * 64) {
    const int hh = idx / D;
    const int d = idx - hh * D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, sml[(ww * 32 + hh) * 2]);
    float A = 0.f, L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float f = fast_exp2(sml[(ww * 32 + hh) * 2] - M);
        A = __builtin_fmaf(so[(ww * 32 + hh) * D + d], f, A);
        L = __builtin_fmaf(sml[(ww * 32 + hh) * 2 + 1], f, L);
      }
    }
    const int rr = row_base + hh;
    const int tt = rr / p.group;
    const int h = kvh * p.group + (rr - tt * p.group);
    if (S == 1) {
      uint16_t* op = reinterpret_cast<uint16_t*>(p.out) + (b * p.o_sb + tt * p.o_st + h * p.o_sh + d);
      *op = Pair<QT>::from_float(L > 0.f ? A / L : 0.f);
    } else {
      const int64_t row = (((int64_t)b * p.T + tt) * p.H + h) * S + split;
      const bool coh = p.counters != nullptr;
      ws_store(p.ws_acc + row * D + d, A, coh);
      if (d == 0) {
        ws_store(p.ws_ml + row * 2 + 0, M, coh);
        ws_store(p.ws_ml + row * 2 + 1, L, coh);
      }
    }
  }
  if (S > 1 && p.counters) {
    merge_in_launch<QT, D>(p, S, nvalid, [&](int j, int64_t& bh, int64_t& o) {
      const int rr = row_base + j;
      const int tt = rr / p.group;
      const int h = kvh * p.group + (rr - tt * p.group);
      bh = ((int64_t)b * p.T + tt) * p.H + h;
      o = (int64_t)b * p.o_sb + (int64_t)tt * p.o_st + (int64_t)h * p.o_sh;
    });
  }
}

// Log-sum-exp merge of split-K partitions (decode.py:316-356 semantics):
//   M = max_s m_s, w_s = 2^(m_s - M), o = sum_s acc_s w_s / sum_s l_s w_s.
// Rows are (sequence, token, head) with T tokens per sequence: one launch
// per decode (decode_merge_kernel), or inside the decode launch by its last
// partition (merge_in_launch), with the same arithmetic.
template <typename QT, int SMAX>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ ws_acc,
                                                           const float* __restrict__ ws_ml, uint8_t* out,
                                                           int B, int T, int H, int D, int S, int64_t o_sb,
                                                           int64_t o_st, int64_t o_sh) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)B * T * H * D) return;
  const int d = idx % D;
  const int64_t bh = idx / D;
  const int h = bh % H;
  const int64_t bt = bh / H;
  const int t = bt % T;
  const int b = bt / T;
  merge_elem<QT, SMAX>(ws_acc, ws_ml, bh, d, D, S, out, (int64_t)b * o_sb + (int64_t)t * o_st + (int64_t)h * o_sh + d);
}

}  // namespace fat

// ===========================================================================
// Host side
// ===========================================================================
namespace {

int ilog2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

template <typename QT, int KV, int D, int HG>
int launch_decode_t(const fat::DecodeParams& prm, int nw, dim3 grid, hipStream_t stream) {
  if (nw == 8) {
    hipLaunchKernelGGL((fat::paged_decode_kernel<QT, KV, D, HG, 8>), grid, dim3(8 * 64), 0, stream, prm);
  } else {
    hipLaunchKernelGGL((fat::paged_decode_kernel<QT, KV, D, HG, 4>), grid, dim3(4 * 64), 0, stream, prm);
  }
  return fat_host::launch_status("paged_decode_kernel");
}

// 8-bit caches take the VALU kernel only with 4-head groups: the 8-head
// instantiations with in-register dequantisation spill (the MFMA kernel is
// the library's choice for 8-bit caches anyway).
template <typename QT, int KV>
int launch_decode_kv(const fat::DecodeParams& prm, int D, int HG, int nw, dim3 grid, hipStream_t stream) {
  if constexpr (KV == fat::KV_SAME) {
    if (HG == 8)
      return D == 128 ? launch_decode_t<QT, KV, 128, 8>(prm, nw, grid, stream)
                      : launch_decode_t<QT, KV, 64, 8>(prm, nw, grid, stream);
  }
  return D == 128 ? launch_decode_t<QT, KV, 128, 4>(prm, nw, grid, stream)
                  : launch_decode_t<QT, KV, 64, 4>(prm, nw, grid, stream);
}

template <typename QT>
int launch_decode_q(const fat::DecodeParams& prm, int kv, int D, int HG, int nw, dim3 grid,
                    hipStream_t stream) {
  switch (kv) {
    case fat::KV_SAME: return launch_decode_kv<QT, fat::KV_SAME>(prm, D, HG, nw, grid, stream);
    case fat::KV_I8: return launch_decode_kv<QT, fat::KV_I8>(prm, D, HG, nw, grid, stream);
    default: return launch_decode_kv<QT, fat::KV_FP8>(prm, D, HG, nw, grid, stream);
  }
}


template <typename QT, int KV, int NW>
void launch_decode_mfma_kvw(const fat::DecodeParams& prm, int D, dim3 grid, hipStream_t stream) {
  if (D == 128)
    hipLaunchKernelGGL((fat::paged_decode_mfma_kernel<QT, KV, 128, NW>), grid, dim3(NW * 64), 0, stream, prm);
  else
    hipLaunchKernelGGL((fat::paged_decode_mfma_kernel<QT, KV, 64, NW>), grid, dim3(NW * 64), 0, stream, prm);
}

template <typename QT, int KV>
void launch_decode_mfma_kv(const fat::DecodeParams& prm, int D, int nw, dim3 grid, hipStream_t stream) {
  if (nw == 8) launch_decode_mfma_kvw<QT, KV, 8>(prm, D, grid, stream);
  else launch_decode_mfma_kvw<QT, KV, 4>(prm, D, grid, stream);
}

template <typename QT>
void launch_decode_mfma_q(const fat::DecodeParams& prm, int kv, int D, int nw, dim3 grid, hipStream_t stream) {
  switch (kv) {
    case fat::KV_SAME: launch_decode_mfma_kv<QT, fat::KV_SAME>(prm, D, nw, grid, stream); break;
    case fat::KV_I8: launch_decode_mfma_kv<QT, fat::KV_I8>(prm, D, nw, grid, stream); break;
    default: launch_decode_mfma_kv<QT, fat::KV_FP8>(prm, D, nw, grid, stream); break;
  }
}

template <typename QT, int SMAX>
void launch_merge_s(const fat::DecodeParams& prm, const fat_decode_args* a, int D, dim3 mgrid, hipStream_t stream) {
  hipLaunchKernelGGL((fat::decode_merge_kernel<QT, SMAX>), mgrid, dim3(256), 0, stream, prm.ws_acc, prm.ws_ml,
                     prm.out, a->batch, prm.T, a->num_heads, D, a->split_k, a->out_stride_b, prm.o_st,
                     a->out_stride_h);
}

template <typename QT>
void launch_merge_q(const fat::DecodeParams& prm, const fat_decode_args* a, int D, dim3 mgrid, hipStream_t stream) {
  const int S = a->split_k;
  if (S <= 4) launch_merge_s<QT, 4>(prm, a, D, mgrid, stream);
  else if (S <= 8) launch_merge_s<QT, 8>(prm, a, D, mgrid, stream);
  else if (S <= 16) launch_merge_s<QT, 16>(prm, a, D, mgrid, stream);
  else if (S <= 32) launch_merge_s<QT, 32>(prm, a, D, mgrid, stream);
  else launch_merge_s<QT, 64>(prm, a, D, mgrid, stream);  // split_k <= 64 (validated)
}

int launch_merge(const fat::DecodeParams& prm, const fat_decode_args* a, int D, hipStream_t stream) {
  const int64_t n = (int64_t)a->batch * prm.T * a->num_heads * D;
  const dim3 mgrid((unsigned)((n + 255) / 256));
  if (a->q_dtype == FAT_DTYPE_F16) launch_merge_q<fat::F16>(prm, a, D, mgrid, stream);
  else if (a->q_dtype == FAT_DTYPE_BF16) launch_merge_q<fat::BF16>(prm, a, D, mgrid, stream);
  else launch_merge_q<fat::F32>(prm, a, D, mgrid, stream);
  return fat_host::launch_status("decode_merge_kernel");
}

}  // namespace

extern "C" size_t fat_paged_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim,
                                                   int32_t split_k) {
  if (split_k <= 1 || batch <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return (size_t)batch * num_heads * split_k * (head_dim + 2) * sizeof(float);
}

// One counter per (query row, head): at least one per (sequence, token
// group, head group) of any kernel's grid.
extern "C" size_t fat_paged_decode_counters_bytes(int32_t rows, int32_t num_heads) {
  if (rows <= 0 || num_heads <= 0) return 0;
  return (size_t)rows * num_heads * sizeof(int32_t);
}

extern "C" int fat_paged_decode(const fat_decode_args* a, void* stream_ptr) {
  fat_host::clear_error();
  if (!a) {
    fat_host::set_error("fat_paged_decode: args is NULL");
    return FAT_E_INVALID;
  }
  if (!a->q || !a->k_cache || !a->v_cache || !a->page_table || !a->seq_lens || !a->out) {
    fat_host::set_error("fat_paged_decode: a required pointer is NULL");
    return FAT_E_INVALID;
  }
  if (a->batch <= 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->num_pages <= 0 || a->max_pages <= 0) {
    fat_host::set_error("fat_paged_decode: batch, heads, num_pages and max_pages must be positive");
    return FAT_E_INVALID;
  }
  if (a->num_heads % a->num_kv_heads != 0) {
    fat_host::set_error("fat_paged_decode: num_heads %d must be divisible by num_kv_heads %d", a->num_heads,
                        a->num_kv_heads);
    return FAT_E_INVALID;
  }
  if (a->split_k < 1 || a->split_k > 64) {
    fat_host::set_error("fat_paged_decode: split_k must be in [1, 64], got %d", a->split_k);
    return FAT_E_INVALID;
  }
  if (a->q_dtype != FAT_DTYPE_F16 && a->q_dtype != FAT_DTYPE_BF16 && a->q_dtype != FAT_DTYPE_F32) {
    fat_host::set_error("fat_paged_decode: q_dtype must be fp16, bf16 or fp32");
    return FAT_E_UNSUPPORTED;
  }
  int kv;
  if (a->kv_dtype == a->q_dtype) kv = fat::KV_SAME;
  else if (a->q_dtype != FAT_DTYPE_F32 && a->kv_dtype == FAT_DTYPE_I8) kv = fat::KV_I8;
  else if (a->q_dtype != FAT_DTYPE_F32 && a->kv_dtype == FAT_DTYPE_FP8E4M3) kv = fat::KV_FP8;
  else {
    fat_host::set_error("fat_paged_decode: kv_dtype must equal q_dtype, or be int8/fp8e4m3 with fp16/bf16 queries");
    return FAT_E_UNSUPPORTED;
  }
  if (kv != fat::KV_SAME && (!a->k_scale || !a->v_scale)) {
    fat_host::set_error("fat_paged_decode: int8/fp8 K/V need k_scale and v_scale");
    return FAT_E_INVALID;
  }
  const int D = a->head_dim;
  if (D < 16 || D > 512 || (D & (D - 1)) != 0) {
    fat_host::set_error("fat_paged_decode: head_dim %d unsupported (a power of two from 16 to 512)", D);
    return FAT_E_UNSUPPORTED;
  }
  if (a->page_size < 1) {
    fat_host::set_error("fat_paged_decode: page_size must be positive, got %d", a->page_size);
    return FAT_E_INVALID;
  }
  const int log2P = ilog2_exact(a->page_size);
  if (a->waves_per_group != 0 && a->waves_per_group != 4 && a->waves_per_group != 8) {
    fat_host::set_error("fat_paged_decode: waves_per_group must be 0 (auto), 4 or 8, got %d", a->waves_per_group);
    return FAT_E_INVALID;
  }
  if (a->pages_per_split < 0) {
    fat_host::set_error("fat_paged_decode: pages_per_split must be >= 0, got %d", a->pages_per_split);
    return FAT_E_INVALID;
  }
  if (a->split_k > 1 && !a->workspace) {
    fat_host::set_error("fat_paged_decode: split_k > 1 needs a workspace");
    return FAT_E_INVALID;
  }
  if ((uintptr_t)a->merge_counters & 3) {
    fat_host::set_error("fat_paged_decode: merge_counters must be 4-byte aligned");
    return FAT_E_INVALID;
  }
  if (a->q_len < 0 || a->q_len > 64) {
    fat_host::set_error("fat_paged_decode: q_len must be in [0, 64] (0 and 1 = one query per sequence), got %d",
                        a->q_len);
    return FAT_E_INVALID;
  }
  const int T = a->q_len > 1 ? a->q_len : 1;
  if (a->kernel != FAT_KERNEL_AUTO && a->kernel != FAT_KERNEL_DECODE_VALU && a->kernel != FAT_KERNEL_DECODE_MFMA &&
      a->kernel != FAT_KERNEL_DECODE_GENERIC) {
    fat_host::set_error("fat_paged_decode: kernel must be FAT_KERNEL_AUTO (0), _DECODE_VALU (1), _DECODE_MFMA (2) "
                        "or _DECODE_GENERIC (3), got %d", a->kernel);
    return FAT_E_INVALID;
  }
  if (a->kernel == FAT_KERNEL_DECODE_VALU && T > 1) {
    fat_host::set_error("fat_paged_decode: the VALU decode kernel takes one query per sequence (q_len %d)", T);
    return FAT_E_UNSUPPORTED;
  }
  // The VALU and MFMA kernels take fp16/bf16 queries, head_dim 64 or 128 and
  // power-of-two pages of at least the rows one 16-byte load per lane covers
  // (their loads read one page id per load); the generic kernel takes the rest.
  const int rpl = (kv == fat::KV_SAME) ? (D == 128 ? 4 : 8) : (D == 128 ? 8 : 16);
  // They address K/V through 32-bit byte offsets from a page's base: strides
  // non-negative, a page below 4 GB, the rows of one 32-key block below 2 GB.
  const int64_t kv_eb = (kv == fat::KV_SAME) ? (a->q_dtype == FAT_DTYPE_F32 ? 4 : 2) : 1;
  auto fits32 = [&](int64_t sp, int64_t ss, int64_t sh) {
    return sp >= 0 && ss >= 0 && sh >= 0 && kv_eb * sp < (int64_t(1) << 32) && kv_eb * (32 * ss + D) < (int64_t(1) << 31);
  };
  const bool strides_ok = fits32(a->k_stride_page, a->k_stride_slot, a->k_stride_head) &&
                          fits32(a->v_stride_page, a->v_stride_slot, a->v_stride_head);
  const bool fast_ok = a->q_dtype != FAT_DTYPE_F32 && (D == 64 || D == 128) && log2P >= 0 && a->page_size >= rpl &&
                       strides_ok;
  const bool generic = a->kernel == FAT_KERNEL_DECODE_GENERIC || (a->kernel == FAT_KERNEL_AUTO && !fast_ok);
  if (!generic && !fast_ok) {
    fat_host::set_error("fat_paged_decode: the %s decode kernel takes fp16/bf16 queries, head_dim 64 or 128, "
                        "power-of-two pages of at least %d rows and non-negative K/V strides with pages below "
                        "4 GB (page_size %d, head_dim %d); use FAT_KERNEL_AUTO or FAT_KERNEL_DECODE_GENERIC",
                        a->kernel == FAT_KERNEL_DECODE_VALU ? "VALU" : "MFMA", rpl, a->page_size, D);
    return FAT_E_UNSUPPORTED;
  }
  if (generic && T > 1) {
    fat_host::set_error("fat_paged_decode: multi-token decode (q_len %d) runs on the MFMA kernel, which takes "
                        "fp16/bf16, head_dim 64 or 128 and power-of-two pages of at least %d rows", T, rpl);
    return FAT_E_UNSUPPORTED;
  }
  // 16-byte alignment of every row start the kernels load.
  const int qeb = a->q_dtype == FAT_DTYPE_F32 ? 4 : 2;
  const int eb = (kv == fat::KV_SAME) ? qeb : 1;
  const uintptr_t q_align = generic ? 0
                                    : ((uintptr_t)a->q | (uintptr_t)(qeb * a->q_stride_b) |
                                       (uintptr_t)(qeb * a->q_stride_h) | (uintptr_t)(T > 1 ? qeb * a->q_stride_t : 0));
  const uintptr_t align_or = q_align | (uintptr_t)a->k_cache | (uintptr_t)a->v_cache |
                             (uintptr_t)(eb * a->k_stride_page) | (uintptr_t)(eb * a->k_stride_slot) |
                             (uintptr_t)(eb * a->k_stride_head) | (uintptr_t)(eb * a->v_stride_page) |
                             (uintptr_t)(eb * a->v_stride_slot) | (uintptr_t)(eb * a->v_stride_head);
  if (align_or & 15) {
    fat_host::set_error("fat_paged_decode: q/K/V base pointers and row strides must be 16-byte aligned");
    return FAT_E_INVALID;
  }

  const int group = a->num_heads / a->num_kv_heads;
  bool use_mfma = group >= fat::kDecMfmaMinGroup || (kv != fat::KV_SAME && FAT_DEC_MFMA_8BIT);
  if (a->kernel == FAT_KERNEL_DECODE_VALU || a->kernel == FAT_KERNEL_DECODE_MFMA)
    use_mfma = a->kernel == FAT_KERNEL_DECODE_MFMA;
  if (T > 1) use_mfma = true;  // only the MFMA kernel has per-token rows
  if (!generic && !use_mfma && kv != fat::KV_SAME && group >= 8) {
    fat_host::set_error("fat_paged_decode: the VALU decode takes int8/fp8 caches for GQA groups below 8 "
                        "(group %d); use FAT_KERNEL_AUTO or FAT_KERNEL_DECODE_MFMA", group);
    return FAT_E_UNSUPPORTED;
  }
  const int HG = generic ? (group < fat_host::kGenericHeads ? group : fat_host::kGenericHeads)
                         : (use_mfma ? 32 : (group >= 8 ? 8 : 4));
  const int hg_per_kv = (group * T + HG - 1) / HG;

  fat::DecodeParams prm{};
  prm.q = static_cast<const uint8_t*>(a->q);
  prm.k = static_cast<const uint8_t*>(a->k_cache);
  prm.v = static_cast<const uint8_t*>(a->v_cache);
  prm.ks = a->k_scale;
  prm.vs = a->v_scale;
  prm.pt = a->page_table;
  prm.lens = a->seq_lens;
  prm.out = static_cast<uint8_t*>(a->out);
  const size_t acc_elems = (size_t)a->batch * T * a->num_heads * a->split_k * D;
  prm.ws_acc = a->split_k > 1 ? static_cast<float*>(a->workspace) : nullptr;
  prm.ws_ml = a->split_k > 1 ? static_cast<float*>(a->workspace) + acc_elems : nullptr;
  prm.q_sb = a->q_stride_b;
  prm.q_sh = a->q_stride_h;
  prm.q_st = T > 1 ? a->q_stride_t : 0;
  prm.k_sp = a->k_stride_page;
  prm.k_ss = a->k_stride_slot;
  prm.k_sh = a->k_stride_head;
  prm.v_sp = a->v_stride_page;
  prm.v_ss = a->v_stride_slot;
  prm.v_sh = a->v_stride_head;
  prm.sc_sp = a->scale_stride_page;
  prm.sc_sh = a->scale_stride_head;
  prm.pt_sb = a->page_table_stride;
  prm.o_sb = a->out_stride_b;
  prm.o_sh = a->out_stride_h;
  prm.o_st = T > 1 ? a->out_stride_t : 0;
  prm.T = T;
  prm.H = a->num_heads;
  prm.Hkv = a->num_kv_heads;
  prm.group = group;
  prm.hg_per_kv = hg_per_kv;
  prm.P = a->page_size;
  prm.log2P = log2P;
  prm.num_pages = a->num_pages;
  prm.max_pages = a->max_pages;
  prm.pps_fixed = a->pages_per_split;
  prm.scale_log2 = a->softmax_scale * fat::kLog2e;
  // Split-K merge inside the decode launch (VALU and MFMA kernels, split_k
  // <= 16) when the caller gives the counters and a workgroup's rows make at
  // most two output elements per thread: the last workgroup of a head group
  // merges alone, so wider groups (e.g. MQA's 32 heads) and more partitions
  // keep the merge kernel, which spreads the elements over many workgroups
  // (measured on MI355X: 32 partitions merged in the launch ran 1-11 %
  // slower, 16 and fewer 2-21 % faster).
  const int S = a->split_k;
  auto use_fused = [&](int rows_per_wg, int nw) {
    return S > 1 && S <= 16 && a->merge_counters != nullptr && rows_per_wg * D <= 2 * 64 * nw;
  };
  bool fused = false;
  prm.counters = nullptr;
  prm.smax = S <= 4 ? 4 : S <= 8 ? 8 : 16;

  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const dim3 grid(a->split_k, a->num_kv_heads * hg_per_kv, a->batch);
  const int64_t wgs = (int64_t)grid.x * grid.y * grid.z;
  const int64_t pages_per_wg =
      a->pages_per_split > 0 ? a->pages_per_split : ((int64_t)a->max_pages + a->split_k - 1) / a->split_k;
  if (generic) {
    const int rc = fat_host::launch_decode_generic(prm, a->q_dtype, kv, D, HG, grid, stream);
    if (rc != FAT_OK || a->split_k == 1) return rc;
    return launch_merge(prm, a, D, stream);
  }
  if (use_mfma) {
    // 8 waves per workgroup pay off only when the grid leaves CUs short of
    // workgroups and each partition is long (>= 2048 keys, measured on
    // MI355X); short partitions finish sooner with 4.
    int nw = a->waves_per_group ? a->waves_per_group
                                : ((wgs < 2 * 256 && pages_per_wg * a->page_size >= 2048) ? 8 : 4);
    fused = use_fused(std::min(32, group * T), nw);
    prm.counters = fused ? a->merge_counters : nullptr;
    if (a->q_dtype == FAT_DTYPE_F16) launch_decode_mfma_q<fat::F16>(prm, kv, D, nw, grid, stream);
    else launch_decode_mfma_q<fat::BF16>(prm, kv, D, nw, grid, stream);
    const int rc = fat_host::launch_status("paged_decode_mfma_kernel");
    if (rc != FAT_OK || a->split_k == 1 || fused) return rc;
    return launch_merge(prm, a, D, stream);
  }
  // 8-wave workgroups keep more loads in flight per CU.  They pay off when
  // fewer than two 4-wave workgroups per CU leave the 256 CUs short of waves,
  // and in any grid when each partition is long (>= 1024 keys: +8-12 % at
  // B128, ctx 1024-16384, measured on MI355X); short partitions in big grids
  // finish sooner with 4.
  const int nw = a->waves_per_group ? a->waves_per_group
                                    : ((wgs < 2 * 256 || pages_per_wg * a->page_size >= 1024) ? 8 : 4);
  fused = use_fused(std::min(HG, group), nw);
  prm.counters = fused ? a->merge_counters : nullptr;
  int rc = (a->q_dtype == FAT_DTYPE_F16) ? launch_decode_q<fat::F16>(prm, kv, D, HG, nw, grid, stream)
                                         : launch_decode_q<fat::BF16>(prm, kv, D, HG, nw, grid, stream);
  if (rc != FAT_OK || a->split_k == 1 || fused) return rc;

  return launch_merge(prm, a, D, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the split-K workspace lives in a file-scope device
// array instead of caller memory.  Every GPU the library runs on holds its
// own copy of `scratch` (kScratchBytes) until the process ends.  Its device
// address is looked up once per device with hipGetSymbolAddress (the array's
// name is only a host-side stand-in) and used for every launch after that.
// Nothing in it needs clearing: each partition of a launch writes its whole
// (acc, m, l) row before the merge reads it.  Two calls that overlap on one
// GPU (different streams) share the array and race.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = FAT_DECODE_NOALLOC_MAX_WORKSPACE;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

}  // namespace

extern "C" int fat_paged_decode_noalloc(const fat_decode_args* a, void* stream) {
  fat_host::clear_error();
  if (!a) {
    fat_host::set_error("fat_paged_decode_noalloc: args is NULL");
    return FAT_E_INVALID;
  }
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fat_host::set_error("fat_paged_decode_noalloc: no current HIP device (or device id >= %d)", kMaxDevices);
    return FAT_E_INVALID;
  }
  // The array is per device: a stream of another device would get this
  // device's address and fault or corrupt there.
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess || sdev != dev) {
      fat_host::set_error("fat_paged_decode_noalloc: the stream belongs to device %d, the current device is %d",
                          (int)sdev, dev);
      return FAT_E_INVALID;
    }
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* ptr = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? ptr : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev]) {
    fat_host::set_error("fat_paged_decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(g_scratch_err[dev]));
    return FAT_E_LAUNCH;
  }
  if (a->batch <= 0 || a->num_heads <= 0 || a->head_dim <= 0 || a->split_k < 1 || a->q_len < 0) {
    return fat_paged_decode(a, stream);  // the regular entry reports the bad argument
  }
  const int64_t rows = (int64_t)a->batch * (a->q_len > 1 ? a->q_len : 1);
  const size_t need = a->split_k > 1 ? (size_t)rows * a->num_heads * a->split_k * (a->head_dim + 2) * sizeof(float)
                                     : 0;
  if (need > kScratchBytes) {
    fat_host::set_error("fat_paged_decode_noalloc: this launch needs %zu bytes of split-K workspace; the "
                        "allocation-free entry holds at most %zu (lower split_k, or use fat_paged_decode with a "
                        "workspace)", need, kScratchBytes);
    return FAT_E_INVALID;
  }
  fat_decode_args b = *a;
  b.workspace = need ? g_scratch_ptr[dev] : nullptr;
  b.merge_counters = nullptr;  // a second kernel merges: no state outside the scratch array
  const int rc = fat_paged_decode(&b, stream);
  if (rc != FAT_OK) {
    // Name this entry in the message the shared path set.
    char msg[480];
    snprintf(msg, sizeof(msg), "%s", fat_last_error());
    fat_host::set_error("fat_paged_decode_noalloc: %s", msg);
  }
  return rc;
}
