// prefill_wide.hip -- the 8-wave ping-pong prefill kernel with 64 query rows
// per wave (512 per workgroup), for long packed sequences at head_dim 128.
//
// Semantics are those of prefill_pp_kernel (prefill.hip) and of
// flashattn_tile/kernels/prefill.py:35-138: online softmax over K/V tiles,
// bottom-right causal masking (query i sees key j iff j <= i + kv_len -
// q_len), P rounded to fp16 for the PV product, fp32 accumulation.
//
// Why a second ping-pong kernel.  In prefill_pp_kernel every wave holds 32
// query rows, so each v_mfma_f32_32x32x16 takes a fresh 1 KB K or V fragment
// from LDS: 256 KB of LDS reads per CU per 64-key tile, as long as the MFMAs
// themselves.  Here each fragment feeds two MFMAs (the wave's two 32-row
// blocks), which halves the LDS bytes per FLOP.  The registers this needs
// (O: 128, Q: 64 per lane) fit the 256 of a wave at two waves per SIMD
// because
//   * tiles are 32 keys, so S^T takes 32 registers and P 16;
//   * the MFMA phase runs O += V(t-1) P(t-1) before S(t) = K(t) Q^T, so P and
//     S are never live at the same time;
//   * K and V tiles go from HBM straight into LDS (gfx950's
//     buffer_load_dwordx4 ... lds: lane i of a load writes 16 bytes at the
//     wave's LDS base + 16 i), with no staging registers and no ds_write.
//
// Ping-pong, as in prefill_pp_kernel: group A (waves 0-3) loads K tiles,
// group B (waves 4-7) V tiles; waves w and w + 4 share a SIMD and run
// opposite phases (MFMAs / softmax), swapped by one workgroup barrier per
// half step.  LDS holds three tiles of K and three of V: while tile t is
// read, t + 1 has landed or is landing and t + 2 is in flight, so a load has
// two half steps to arrive.  A wave waits for its own loads (vmcnt) before
// the barrier after which other waves read them.
//
// LDS tile layout: 32 rows, padded so that the MFMA operand reads hit
// distinct banks with plain immediate offsets: K rows every 272 bytes
// (ds_read_b128 of 16 rows at one chunk: 4-bank groups (li + c) mod 16), V
// rows every 320 bytes (ds_read_b64_tr_b16 of 4 rows x 4 chunks per 32
// lanes: banks 16 tc + 4 c + 2 h).  A load writes 64 consecutive 16-byte
// slots; a lane whose slot is a row's padding is masked off, the others fetch
// their slot's chunk.  Rows past kv_len lie past the buffer descriptor's
// range and arrive as zeros.
//
// bf16: only with V converted to fp16 ahead of the kernel (the pre-pass in
// prefill.hip, one power-of-two scale 2^-s per (sequence, KV head)): QK^T
// runs as bf16 MFMAs, PV as fp16 ones on that copy, and O = acc * 2^s / l.
#include "prefill_common.h"

namespace fat {

constexpr int kWideRows = 64;   // query rows per wave
constexpr int kWideBN = 32;     // keys per tile
constexpr int kWideBufs = 3;    // LDS tiles per stream
constexpr int kKSlots = 17;     // 16-byte slots per K row (16 + 1 padding)
constexpr int kVSlots = 20;     // 16-byte slots per V row (16 + 4 padding)
constexpr int kKTile = kWideBN * kKSlots * 16;  // 8704 bytes
constexpr int kVTile = kWideBN * kVSlots * 16;  // 10240 bytes
constexpr int kVArea = kWideBufs * kKTile;      // the V tiles follow the K tiles
static_assert(kWideBM == 8 * kWideRows, "workgroup rows");

// MFMA-phase schedule: NPV entries of O += V P (two transposed reads, two
// MFMAs each), then NE - NPV entries of S = K Q^T (one read, two MFMAs
// each); the reads of entry e + LOOK issue right after entry e's MFMAs.
template <int E, int LOOK, int NE, int NPV>
struct WideReads {
  static __device__ __forceinline__ void apply() {
    if constexpr (E < LOOK && E < NE) {
      __builtin_amdgcn_sched_group_barrier(0x100, E < NPV ? 2 : 1, 0);
      WideReads<E + 1, LOOK, NE, NPV>::apply();
    }
  }
};
template <int E, int NE, int NPV, int LOOK>
struct WideOrder {
  static __device__ __forceinline__ void apply() {
    if constexpr (E == 0) WideReads<0, LOOK, NE, NPV>::apply();
    if constexpr (E < NE) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      if constexpr (E + LOOK < NE) __builtin_amdgcn_sched_group_barrier(0x100, (E + LOOK) < NPV ? 2 : 1, 0);
      WideOrder<E + 1, NE, NPV, LOOK>::apply();
    }
  }
};

// MFMA-phase operand lookahead: entries (two MFMAs each) whose LDS reads are
// in flight ahead of their MFMAs.  2 measured fastest; 1, 3 and 4 ran 4 %
// slower (with 3 or 4 the compiler's register assignment serialises the V
// reads).
#ifndef FAT_WIDE_LOOK
#define FAT_WIDE_LOOK 2
#endif

typedef __attribute__((address_space(3))) void lds_void;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// 16 bytes per lane from buffer `desc` at byte offset `voff` straight into
// LDS at `lds_addr` + 16 * lane (lds_addr wave-uniform, in M0).  Offsets past
// the descriptor's range arrive as zeros.  An SALU write of M0 needs one wait
// state before a load that writes LDS (the s_nop).  Nothing else in the
// kernel keeps a value in M0.
__device__ __forceinline__ void buffer_load_lds16(const i32x4& desc, int voff, int lds_addr) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(desc), "s"(lds_addr)
      : "memory", "m0");
}

// Longest-first order of a packed launch's work items.  Item i = (query
// block jb = i / B counted from the sequence's end, sequence b = i % B); its
// causal chain holds kv_len - 512 jb keys (kv_len when not causal).  Items
// are ordered by chain length (descending), then sequence, then block; items
// without query rows come last.  Each thread ranks one item with a count per
// sequence (a sequence's chains form an arithmetic progression), O(B) work,
// and the workgroup takes the item of rank `target`, or -1 (no rows: the
// workgroup exits).  Needs B * nqb <= blockDim.x and a 2 B + 1 int LDS area;
// every thread of the workgroup calls it.
template <bool CAUSAL>
__device__ __forceinline__ int wide_ranked_item(const PrefillParams& p, int n, int target, int* s_len) {
  constexpr int BM = kWideBM;
  const int t = threadIdx.x;
  const int B = p.B;
  if (t < B) {
    s_len[2 * t] = p.cu_q[t + 1] - p.cu_q[t];
    s_len[2 * t + 1] = p.cu_k[t + 1] - p.cu_k[t];
  }
  if (t == 0) s_len[2 * B] = -1;
  __syncthreads();
  if (t < n) {
    const int tb = t % B;
    const int tj = t / B;
    if (tj * BM < s_len[2 * tb]) {  // the item has query rows
      const int kl = s_len[2 * tb + 1];
      const int X = CAUSAL ? kl - tj * BM : kl;
      int rank = 0;
      for (int b2 = 0; b2 < B; ++b2) {
        const int nb2 = (max(s_len[2 * b2], 0) + BM - 1) / BM;  // items of b2 with rows
        const int kl2 = s_len[2 * b2 + 1];
        if (CAUSAL) {
          // b2's block j2 has chain kl2 - j2 BM: longer than X for j2 < d / BM.
          const int d = kl2 - X;
          rank += d > 0 ? min((d + BM - 1) / BM, nb2) : 0;
          // an equal chain (j2 = d / BM) comes first when b2 < tb
          if (b2 < tb && d >= 0 && d % BM == 0 && d / BM < nb2) ++rank;
        } else {
          if (kl2 > X || (kl2 == X && b2 < tb)) rank += nb2;
          else if (kl2 == X && b2 == tb) rank += tj;
        }
      }
      if (rank == target) s_len[2 * B] = t;
    }
  }
  __syncthreads();
  return s_len[2 * B];
}

template <typename T, bool CAUSAL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_wide_kernel(const PrefillParams p) {
  constexpr int D = 128;
  constexpr int KS = D / 16;  // k-steps of S^T = K Q^T
  constexpr int DB = D / 32;  // 32-row blocks of O^T
  constexpr bool VH = std::is_same<T, BF16>::value;
  // Three K and three V tiles during the loop; eight waves' 32-row output
  // staging areas in the epilogue.
  __shared__ __attribute__((aligned(1024))) uint8_t lds[8 * kOutStage<D> * 2];
  static_assert(kWideBufs * (kKTile + kVTile) <= (int)sizeof(lds), "tiles");

  // Query blocks are counted from each sequence's last row (block jb holds
  // rows [q_len - 512 (jb + 1), q_len - 512 jb)), so a sequence's partly
  // empty block is its first, whose causal chain is the shortest.  The grid
  // runs item (jb, b) = blockIdx.x / H, jb-major (every sequence's longest
  // chain first), or, with rank_items, the items longest chain first
  // (wide_ranked_item); the H query heads of an item are consecutive.
  __shared__ int s_items[2 * kWideRankMaxSeqs + 1];
  int item = blockIdx.x / p.H;
  const int j = blockIdx.x - item * p.H;
  if (p.rank_items > 0) {
    item = wide_ranked_item<CAUSAL>(p, p.rank_items, item, s_items);
    if (item < 0) return;  // uniform: no item of this rank has rows
  }
  const int jb = item / p.B;
  const int b = item - jb * p.B;
  const int kvh = j % p.Hkv;
  const int h = kvh * p.group + j / p.Hkv;

  const int q_start = p.cu_q[b];
  const int q_len = p.cu_q[b + 1] - q_start;
  const int k_start = p.cu_k[b];
  const int kv_len = p.cu_k[b + 1] - k_start;
  if (jb * kWideBM >= q_len) return;  // uniform over the workgroup
  const int r_end = q_len - jb * kWideBM;  // one past the block's last row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;  // 0: group A (loads K), 1: group B (loads V)
  const int wg = w & 3;
  const int g = lane >> 5;
  const int li = lane & 31;
  const int shift = kv_len - q_len;
  // The wave's first row; negative in a sequence's first block when q_len is
  // not a multiple of 512 (rows below 0 compute as row 0 and are not stored).
  const int row0 = r_end - kWideBM + w * kWideRows;
  const float c = p.scale_log2;

  int hi = kv_len;
  if (CAUSAL) hi = min(kv_len, r_end + shift);
  const int n_tiles = hi > 0 ? (hi + kWideBN - 1) / kWideBN : 0;

  f32x16 acc[2][DB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb][db][r] = 0.f;
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};
  const int e_acc = VH ? p.v_head_scale[b * p.Hkv + kvh] : 0;  // bf16: O = acc * 2^e_acc

  // This group's stream: K rows (A) or fp16 V rows (B) of the sequence's KV
  // head, through one buffer descriptor whose range ends with row kv_len - 1.
  const int st = grp ? (int)p.v_st : (int)p.k_st;
  const int st2 = 2 * st;
  const int64_t sh = grp ? p.v_sh : p.k_sh;
  const uint8_t* seq = (grp ? p.v : p.k) + 2 * ((int64_t)k_start * st + (int64_t)kvh * sh);
  const int rec = (int)min((int64_t)max(kv_len - 1, 0) * st2 + 2 * D, (int64_t)0x7fffffff);
  // Loads: a tile is 32 rows of `rs` 16-byte slots (rs = 17 for K, 20 for
  // V), 9 (K) or 10 (V) loads of 64 slots; wave wg of the group takes loads
  // wg, wg + 4 and wg + 8.  Slot s holds chunk s % rs of row s / rs; a lane
  // whose slot is padding or past the tile is masked off.
  const int rs = grp ? kVSlots : kKSlots;
  const int nload = grp ? 10 : 9;             // 64-slot loads per tile
  const int my_loads = (nload - wg + 3) / 4;  // this wave's share: 2 or 3
  const int tile_bytes = grp ? kVTile : kKTile;
  // LDS byte address of this group's buffer 0.
  const int my_area = (int)(uintptr_t)(lds_void*)lds + (grp ? kVArea : 0);
  // The same descriptor as four wave-uniform dwords: base address, stride 0,
  // range, flags.
  const uint64_t seq_addr = reinterpret_cast<uint64_t>(seq);
  const i32x4 desc = {__builtin_amdgcn_readfirstlane((int)(uint32_t)seq_addr),
                      __builtin_amdgcn_readfirstlane((int)((uint32_t)(seq_addr >> 32) & 0xffffu)),
                      __builtin_amdgcn_readfirstlane(rec), kBufFlags};
  // The loads are written as inline asm: the compiler does not track LDS
  // written by a load, so it would otherwise wait for every outstanding load
  // (vmcnt(0)) before each LDS read.  The kernel orders them itself: a
  // wave's own waits (wait_loads), then a workgroup barrier.
  auto issue = [&](int t, int buf) __attribute__((always_inline)) {
    const int toff = t * kWideBN * st2;
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int i = wg + 4 * u;
      if (i < nload) {  // wave-uniform
        const int slot = 64 * i + lane;
        const int r = slot / rs;
        const int ch = slot - r * rs;
        if (ch < 16 && r < kWideBN)
          buffer_load_lds16(desc, r * st2 + 16 * ch + toff, my_area + buf * tile_bytes + 1024 * i);
      }
    }
  };
  // Q of the wave's two 32-row blocks (the B operands of S^T = K Q^T), then
  // the first tile loads, so that their latencies overlap.  The compiler
  // waits for the Q loads before their first use; the tile loads, issued
  // later, only make its in-order vmcnt waits stricter.
  u32x4 qf[2][KS];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int qr = max(row0 + 32 * rb + li, 0);
    const uint8_t* qp = p.q + 2 * ((int64_t)(q_start + qr) * p.q_st + (int64_t)h * p.q_sh + 8 * g);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[rb][ks] = (*reinterpret_cast<const u32x4*>(qp + 32 * ks) & p.q_and) ^ p.q_xor;
  }
  if (n_tiles > 0) issue(0, 0);
  // Wait until this wave's loads of every tile before the most recent issue
  // have landed (`pending`: that issue's my_loads loads may still be in flight).
  auto wait_loads = [&](bool pending) __attribute__((always_inline)) {
    if (!pending) __builtin_amdgcn_s_waitcnt(0x0F70);
    else if (my_loads == 3) __builtin_amdgcn_s_waitcnt(0x0F73);
    else __builtin_amdgcn_s_waitcnt(0x0F72);
  };

  // Operand addresses: one per-lane base plus immediates.  K: lane (li, g)
  // reads row li, chunk 2 ks + g.  V^T through ds_read_b64_tr_b16: in each
  // 16-lane group G, lane (tc, tj) reads 8 bytes of row 16 tt + 4 (G / 2) + tc
  // (and that + 8) at columns 32 db + 16 (G % 2) + 4 tj.
  const int tr_G = lane >> 4;
  const int tr_c = (lane & 15) >> 2;
  const int tr_j = lane & 3;
  const int kbase = li * (kKSlots * 16) + 16 * g;
  const int vbase = kVArea + (4 * (tr_G >> 1) + tr_c) * (kVSlots * 16) + 32 * (tr_G & 1) + 8 * tr_j;

  f32x16 s[2];
  u32x4 pf[2][2];

  // S(t) = K(t) Q^T for both row blocks; each K fragment feeds two MFMAs.
  auto qk = [&](int buf) __attribute__((always_inline)) {
    const uint8_t* Kb = lds + kbase + buf * kKTile;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(Kb + 32 * ks);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        if (ks == 0) s[rb] = Mfma<T>::mma(a, qf[rb][0], f32x16{});
        else s[rb] = Mfma<T>::mma(a, qf[rb][ks], s[rb]);
      }
    }
  };
  // O += V(t) P(t) for both row blocks; each V^T fragment feeds two MFMAs.
  auto pv = [&](int buf) __attribute__((always_inline)) {
    const uint16_t* Vb = reinterpret_cast<const uint16_t*>(lds + vbase + buf * kVTile);
    constexpr int RE = kVSlots * 8;  // V row stride, elements
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x2 lo = lds_read_tr16(Vb + 16 * tt * RE + 32 * db);
        const u32x2 hi2 = lds_read_tr16(Vb + (16 * tt + 8) * RE + 32 * db);
        const u32x4 a = {lo[0], lo[1], hi2[0], hi2[1]};
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) acc[rb][db] = Mfma<F16>::mma(a, pf[rb][tt], acc[rb][db]);
      }
  };

  // Softmax of S(t) -> P(t).  P = 2^(s c - m_run) against the running max
  // (no row max) while every partial row sum stays <= 2^kLazyPP.  Otherwise
  // (and on the first tile) the exact path takes the row max, moves m_run
  // when the max exceeds it by more than kLazyPP (rescaling O and l), and
  // computes P again; S(t) is then recomputed from the K tile, still in LDS,
  // since the fast path lets S die as P is formed.
  auto prep = [&](int t) __attribute__((always_inline)) {  // mask S(t)
    const int n0 = t * kWideBN;
    const bool need_mask = (n0 + kWideBN > kv_len) || (CAUSAL && n0 + kWideBN - 1 > row0 + shift);
    if (need_mask) {
      // Element r of this lane holds key n0 + 4 g + (r & 3) + 8 (r >> 2):
      // compared as a constant against lim - n0 - 4 g (constants keep the
      // compiler from holding 16 per-lane key indices across the loop).
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int lim = CAUSAL ? min(kv_len - 1, max(row0 + 32 * rb + li, 0) + shift) : kv_len - 1;
        const int rel = lim - n0 - 4 * g;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[rb][r] = ((r & 3) + 8 * (r >> 2)) <= rel ? s[rb][r] : -INFINITY;
      }
    }
  };
  const float cm = c;  // positive: a non-positive scale is folded into Q
  auto compute_p = [&](int rb) __attribute__((always_inline)) -> float {
    const float nm = -m_run[rb];
    float lsq[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const float x0 = fast_exp2(__builtin_fmaf(s[rb][8 * tt + 2 * e2], cm, nm));
        const float x1 = fast_exp2(__builtin_fmaf(s[rb][8 * tt + 2 * e2 + 1], cm, nm));
        pf[rb][tt][e2] = Pair<F16>::pack(x0, x1);
        if (e2 == 0) lsq[tt] = x0 + x1;
        else lsq[tt] += x0 + x1;
      }
    return lsq[0] + lsq[1];
  };
  auto exact_p = [&]() __attribute__((always_inline)) {
    float ls[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[rb][r]);
      mx = xor32<OpMax>(mx);
      mx *= c;
      const bool grow = mx > m_run[rb] + kLazyPP;
      if (__any(grow)) {
        const float alpha = grow ? fast_exp2(m_run[rb] - mx) : 1.f;
        m_run[rb] = grow ? mx : m_run[rb];
        l_run[rb] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[rb][db][r] *= alpha;
      }
      ls[rb] = compute_p(rb);
    }
    l_run[0] += ls[0];
    l_run[1] += ls[1];
  };
  auto softmax = [&](int t, int kbuf) __attribute__((always_inline)) {
    prep(t);
    if (t == 0) {
      exact_p();
      return;
    }
    const float ls0 = compute_p(0);
    const float ls1 = compute_p(1);
    if (__any(!(ls0 <= kLazyPPSum) || !(ls1 <= kLazyPPSum))) {  // rare; also catches inf / NaN
      qk(kbuf);
      prep(t);
      exact_p();
      return;
    }
    l_run[0] += ls0;
    l_run[1] += ls1;
  };

  if (n_tiles > 0) {
    // Tile t lives in LDS buffer t % 3.  A wave's half step for tile t
    // issues the loads of tile t + 2 and, before its next barrier, waits for
    // its loads of tile t + 1.  Group B runs one barrier behind group A, so
    // the two waves of each SIMD are in opposite phases; every wave passes
    // 2 n_tiles + 2 barriers.
    auto stage = [&](int t, int buf2) __attribute__((always_inline)) {  // buf2 = (t + 2) % 3
      if (t + 2 < n_tiles) issue(t + 2, buf2);
    };
    auto stage_wait = [&](int t) __attribute__((always_inline)) {
      if (t + 1 < n_tiles) wait_loads(t + 2 < n_tiles);
    };
    if (grp == 0) {  // tile 0 was issued with the Q loads
      stage(-1, 1);
      stage_wait(-1);
    }
    if (grp == 1) {
      __syncthreads();
      stage(-1, 1);
      stage_wait(-1);
    }
    __syncthreads();
    qk(0);
    __syncthreads();
    stage(0, 2);
    softmax(0, 0);
    stage_wait(0);
    // Causal: tiles past this wave's last visible key are fully masked for
    // it; from tile nv on the wave only loads tiles and keeps the barrier
    // count.  A wave whose rows all lie before the sequence's first query
    // stops computing after tile 0 (nothing it computes is stored).
    const int nv = row0 + kWideRows <= 0 ? 1
                   : CAUSAL          ? min(n_tiles, (row0 + kWideRows - 1 + shift) / kWideBN + 1)
                                     : n_tiles;
    int bk = 1;  // t % 3 for the loop's t
    for (int t = 1; t < nv; ++t) {
      const int bprev = bk == 0 ? 2 : bk - 1;  // (t - 1) % 3 == (t + 2) % 3
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(2);
      pv(bprev);
      qk(bk);
      WideOrder<0, 4 * DB / 2 + KS, 2 * DB, FAT_WIDE_LOOK>::apply();
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      stage(t, bprev);
      softmax(t, bk);
      stage_wait(t);
      bk = bk == 2 ? 0 : bk + 1;
    }
    __syncthreads();
    pv((nv - 1) % 3);
    for (int t = nv; t < n_tiles; ++t) {
      __syncthreads();
      stage(t, (t + 2) % 3);
      stage_wait(t);
      __syncthreads();
    }
    if (grp == 0) __syncthreads();
  }

  // Epilogue: each wave stages its two 32-row blocks in turn in its own
  // area, once every wave is done with the tiles.
  __syncthreads();
  uint16_t* ob = reinterpret_cast<uint16_t*>(lds) + w * kOutStage<D>;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    if (rb == 1) wave_lds_fence();  // block 0's reads of the area precede block 1's writes
    write_rows_via_lds<T, D, DB>(ob, li, g, lane, acc[rb], l_run[rb], e_acc, VH, p, q_start, q_len, h,
                                 row0 + 32 * rb);
  }
}

}  // namespace fat

namespace fat_host {

template <typename T, bool CAUSAL>
static void launch_wide_c(const fat::PrefillParams& prm, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((fat::prefill_wide_kernel<T, CAUSAL>), grid, dim3(512), 0, stream, prm);
}

int launch_prefill_wide(const fat::PrefillParams& prm, bool bf16, bool causal, dim3 grid, hipStream_t stream) {
  if (bf16) {
    if (causal) launch_wide_c<fat::BF16, true>(prm, grid, stream);
    else launch_wide_c<fat::BF16, false>(prm, grid, stream);
  } else {
    if (causal) launch_wide_c<fat::F16, true>(prm, grid, stream);
    else launch_wide_c<fat::F16, false>(prm, grid, stream);
  }
  return launch_status("prefill_wide_kernel");
}

}  // namespace fat_host
