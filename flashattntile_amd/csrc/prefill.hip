// prefill.hip -- packed varlen flash-attention forward for gfx950 (CDNA4 MFMA).
//
// Behaviour follows flashattn_tile/kernels/prefill.py:35-138
// (_fwd_varlen_kernel): per (query block, query head, sequence) it streams
// K/V blocks, keeps a running max / sum / fp32 accumulator (online softmax),
// applies bottom-right causal masking (query i sees key j iff
// j <= i + kv_len - q_len) and writes q.dtype.
//
// MI355X design (not a translation of the Triton program):
//   * three kernels, chosen per launch from the grid size and the longest
//     key chain (launch_prefill): prefill_pp_kernel, 8 waves x 32 query rows
//     (256 rows) whose two 4-wave groups run MFMA and softmax phases in
//     ping-pong on each SIMD, for grids that cover the CUs;
//     prefill_kernel<NG = 1>, 4 waves x 32 rows (BM = 128), for smaller
//     grids; prefill_kernel<NG = 2>, two such groups on the same 128 rows
//     taking alternate key tiles (merged through LDS at the end), for grids
//     that leave CUs idle;
//   * K/V blocks of BN = 64 keys are staged in LDS in their natural
//     [key][dim] layout and shared by the waves; the next blocks are
//     prefetched into registers while the current one is computed;
//   * scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_{f16,bf16}: the accumulator then holds one query
//     per lane (column) and 32 keys per lane pair, so the softmax row max /
//     sum need a single lane^32 exchange and the O accumulator is rescaled
//     lane-locally;
//   * O^T = V^T P^T: P^T is the B operand straight from the S^T accumulator
//     registers (the key order inside an MFMA k-step is chosen to match the
//     accumulator layout), and V^T comes from LDS through
//     ds_read_b64_tr_b16, so V never needs a transposed copy;
//   * P is rounded to fp16 for the PV product (prefill.py:128 rounds it to
//     the input dtype).  For bf16 inputs both kernels stage V as fp16, each
//     staging wave's rows scaled by a power of two that is 1 unless some
//     |v| >= 2^15, and fold the scales into P's exponent: the result stays
//     within fp32-level error of the fp32 reference (at most max|v| * 2^-39
//     per V element once |v| reaches 2^15);
//   * exp is 2^(x * log2 e) on v_exp_f32;
//   * the 1-D grid walks query blocks longest-first (causal balance) and
//     assigns the query heads that share a KV head to the same XCD
//     (workgroup id mod 8), so K/V blocks are reused from that XCD's L2;
//   * paged instantiations (PG != 0: fat_prefill_paged, chunked prefill) read
//     K/V through a page table from an NHD page pool instead of packed rows:
//     key j of sequence b is slot j % P of page page_table[b, j / P], and
//     kv_len is seq_lens[b].  Page ids are loaded one tile ahead, so the
//     table lookup is off the load's critical path.  When a page holds at
//     least the rows of one 16-byte-per-lane load (PG 2, PG 3) the page id is
//     wave-uniform and a load is a scalar base plus a constant lane offset
//     (PG 3: one pool descriptor and a 32-bit offset, when every row of the
//     pool lies within 2^31 bytes); otherwise (PG 1) each lane forms its own
//     64-bit address.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "prefill_common.h"

namespace fat {

// Rows of a K or V stream read through the page table.  A lane loads LOADS
// 16-byte chunks per tile, at rows row0 + u * RPL (u < LOADS) of the tile and
// byte column `col`.  The page ids a load needs are fetched by the previous
// load of the same stream (a stream loads every tstep-th tile, in increasing
// order), so the table lookup latency hides behind a whole tile of compute.
template <int LOADS, int RPL>
struct PagedRows {
  const uint8_t* base;  // cache + this KV head's offset
  const int32_t* pt_row;
  int64_t sp2;          // page stride, bytes
  int64_t st2;          // slot stride, bytes
  int pshift, pmask, kv_last, page_last, row0, col;
  int tstep = 1;  // tile distance between this stream's consecutive loads
  int pg[LOADS];

  __device__ __forceinline__ int row_of(int tile, int u) const {
    return min(tile * kBN + row0 + u * RPL, kv_last);
  }
  // Page ids of `tile` into pg (clamped into the pool: a bad table entry
  // reads a wrong page, never outside the allocation).
  __device__ __forceinline__ void fetch_ids(int tile) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) pg[u] = min(max(pt_row[row_of(tile, u) >> pshift], 0), page_last);
  }
  // The chunks of `tile` (its ids already in pg), then the ids of the
  // stream's next tile, tile + tstep.
  __device__ __forceinline__ void load(int tile, u32x4 (&dst)[LOADS]) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int j = row_of(tile, u);
      dst[u] = *reinterpret_cast<const u32x4*>(base + (int64_t)pg[u] * sp2 + (int64_t)(j & pmask) * st2 + col);
    }
    fetch_ids(tile + tstep);
  }
};

// The same streams when page_size >= RPL: the RPL rows of one load then lie
// in one page, so its page id and the row base are wave-uniform (SGPRs) and
// a lane adds only its constant offset -- no per-load vector address math.
// Rows at or past kv_len (last tile only) read slots of the last page and
// are zeroed before they reach LDS (mask_tail).
// OFF32 (PG 3): the pool of this KV head lies within 2^31 bytes of its
// first row, so it is one buffer and a load passes its row's byte offset as
// the 32-bit scalar offset (page * page stride + slot * slot stride): one
// multiply-add per load instead of a 64-bit address and a descriptor.
template <int LOADS, int RPL, bool OFF32 = false>
struct PagedRowsU {
  const uint8_t* base;
  const int32_t* pt_row;
  int64_t sp2, st2;
  int pshift, pmask, kv_len, last_idx, page_last, row0;
  uint32_t lane_off;  // row0 * st2 + col
  int pg[LOADS];      // page ids of the next tile (scalar registers)
  int cur;            // tile whose chunks are in the registers
  int tstep = 1;      // tile distance between this stream's consecutive loads
  __amdgpu_buffer_rsrc_t pool;  // OFF32: the KV head's pool from its first row

  __device__ __forceinline__ void init_pool(int num_pages) {
    (void)num_pages;  // the host checked every row offset against 2^31
    if constexpr (OFF32) pool = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7fffffff, kBufFlags);
  }

  __device__ __forceinline__ int idx(int tile, int u) const {
    return min((tile * kBN + u * RPL) >> pshift, last_idx);
  }
  // The table row is read-only for the kernel's lifetime, so its entries are
  // read through the constant address space: uniform s_load_dword into SGPRs.
  __device__ __forceinline__ void fetch_ids(int tile) {
    const __attribute__((address_space(4))) int32_t* t =
        (const __attribute__((address_space(4))) int32_t*)pt_row;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) pg[u] = t[idx(tile, u)];
  }
  // Each load is a buffer load whose descriptor base is the (uniform) row
  // address and whose 32-bit lane offset is constant: no vector address math.
  __device__ __forceinline__ void load(int tile, u32x4 (&dst)[LOADS]) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int page = min(max(pg[u], 0), page_last);
      const int slot0 = (tile * kBN + u * RPL) & pmask;
      if constexpr (OFF32) {
        const uint32_t so = (uint32_t)page * (uint32_t)sp2 + (uint32_t)slot0 * (uint32_t)st2;
        dst[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(pool, (int)lane_off, (int)so, 0));
      } else {
        const uint8_t* row_base = base + (int64_t)page * sp2 + (int64_t)slot0 * st2;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)row_base, (short)0, 0x7fffffff, kBufFlags);
        dst[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)lane_off, 0, 0));
      }
    }
    cur = tile;
    fetch_ids(tile + tstep);
  }
  __device__ __forceinline__ void mask_tail(u32x4 (&dst)[LOADS]) const {
    if (cur * kBN + kBN > kv_len) {  // wave-uniform
#pragma unroll
      for (int u = 0; u < LOADS; ++u)
        if (cur * kBN + u * RPL + row0 >= kv_len) dst[u] = u32x4{0u, 0u, 0u, 0u};
    }
  }
};

// bf16 V rows held by this wave (LOADS 16-byte chunks per lane) -> fp16,
// scaled by 2^-s with s = max(0, e - 141) for the wave's largest bf16
// exponent field e (inf / NaN: 255), so every |v| 2^-s < 2^15 is exact in
// fp16 up to fp16 subnormals.  Returns s (wave-uniform; 0 unless some
// |v| >= 2^15).
template <int LOADS>
__device__ __forceinline__ int bf16_to_f16_scaled(u32x4 (&reg)[LOADS]) {
  u16x2 em = {0, 0};
#pragma unroll
  for (int u = 0; u < LOADS; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) em = __builtin_elementwise_max(em, __builtin_bit_cast(u16x2, reg[u][e] & 0x7f807f80u));
  const int le = (int)(max(em[0], em[1]) >> 7);
  int sw = 0;
  if (__builtin_amdgcn_ballot_w64(le > 141) != 0) {  // rare: some |v| >= 2^15
    float m = (float)le;
    m = within_quad<OpMax, 4>(m);
    m = across_rows<OpMax, 4>(m);
    sw = __builtin_amdgcn_readfirstlane(max(0, (int)m - 141));
  }
  if (sw == 0) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const u32 wv = reg[u][e];
        reg[u][e] = Pair<F16>::pack(Pair<BF16>::lo(wv), Pair<BF16>::hi(wv));
      }
  } else {
    const float f = as_f32((u32)(127 - sw) << 23);  // 2^-sw, sw <= 114
#pragma unroll
    for (int u = 0; u < LOADS; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const u32 wv = reg[u][e];
        reg[u][e] = Pair<F16>::pack(Pair<BF16>::lo(wv) * f, Pair<BF16>::hi(wv) * f);
      }
  }
  return sw;
}

// For the V tile whose staging waves wrote their scales to sc[0..3]: moves
// O = acc * 2^e_acc to the tile's largest scale if that is larger (rare),
// then gives each (k-step tt, element half hh) of this lane its exponent
// offset o = s_wave - e_acc <= 0 and the factor 2^-o that scales its
// partial row sum back.  Element (tt, e2) of a lane in k-group g holds key
// 4g + 8(2tt + e2/2) + (0..3) of its 32-key block, staged by wave
// (key mod (256/CPR)) / (64/CPR).
template <int CPR, int DB>
__device__ __forceinline__ void v_scale_offsets(const int* sc, int g, int& e_acc, f32x16 (&acc)[DB],
                                                float (&off)[2][2], float (&back)[2][2]) {
  const u32x4 sc4 = *reinterpret_cast<const u32x4*>(sc);
  int sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sv[i] = __builtin_amdgcn_readfirstlane((int)sc4[i]);
  const int smax = max(max(sv[0], sv[1]), max(sv[2], sv[3]));
  if (smax > e_acc) {  // rare: a tile with larger |v| than any before
    const float down = as_f32((u32)(127 - (smax - e_acc)) << 23);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] *= down;
    e_acc = smax;
  }
  constexpr int kRowsPerLoad = 256 / CPR;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int wl = ((4 * g + 8 * (2 * tt + hh)) % kRowsPerLoad) / (64 / CPR);
      const int sws = wl == 0 ? sv[0] : wl == 1 ? sv[1] : wl == 2 ? sv[2] : sv[3];
      off[tt][hh] = (float)(sws - e_acc);
      back[tt][hh] = as_f32((u32)(127 + e_acc - sws) << 23);
    }
}

// A row's running max is only moved (and O rescaled) when a tile's max
// exceeds it by more than this many log2 units; p = 2^(x - m) then stays
// below 2^kLazy, which fp16/bf16 P and the fp32 sums hold exactly as well.
constexpr float kLazy = 8.0f;
#ifndef FAT_PF_PP_MIN_FULL
#define FAT_PF_PP_MIN_FULL 256
#endif
#ifndef FAT_PF_PP_MIN_CAUSAL
#define FAT_PF_PP_MIN_CAUSAL 256
#endif
#ifndef FAT_PF_WIDE_MIN_FULL
#define FAT_PF_WIDE_MIN_FULL 256
#endif
#ifndef FAT_PF_WIDE_MIN_CAUSAL
#define FAT_PF_WIDE_MIN_CAUSAL 256
#endif
#ifndef FAT_PF_WIDE_MEAN
#define FAT_PF_WIDE_MEAN 2048
#endif
#ifndef FAT_PF_SPLIT_MAX
#define FAT_PF_SPLIT_MAX 256
#endif
#ifndef FAT_PF_SPLIT_TILES
#define FAT_PF_SPLIT_TILES 8
#endif
#ifndef FAT_PF_SPLIT_LONG
#define FAT_PF_SPLIT_LONG 32
#endif

// The scale c is positive (launch_prefill folds a negative or zero
// softmax scale into Q), so max_j(s_j * c) = c * max_j(s_j) and the scale is
// folded into the exponent's fma.
// NG = 2: two groups of 4 waves take alternate K/V tiles for the same query
// rows (group g tiles g, g + 2, ...) and merge (m, l, O) through LDS at the
// end, halving the tile chain of a query block: for grids too small to
// give every CU more than one workgroup.
// D = 256 (NG = 1 only) holds O (128 registers) and Q (64) per lane and runs
// one wave per SIMD with up to 512 registers.
template <typename T, int D, bool CAUSAL, int PG, int NG>
__global__ __launch_bounds__(256 * NG)
__attribute__((amdgpu_waves_per_eu(D >= 256 ? 1 : 2, D >= 256 ? 1 : 2)))
void prefill_kernel(const PrefillParams p) {
  constexpr int KS = D / 16;        // MFMA k-steps of S^T over the head dim
  constexpr int DB = D / 32;        // 32-row blocks of O^T
  constexpr int K_RS = D + 8;       // LDS row strides (elements), chosen to
  constexpr int V_RS = D + 32;      // spread 16-byte / transposed reads over banks
  constexpr int CPR = D / 8;        // 16-byte chunks per K/V row
  constexpr int LOADS = kBN * CPR / 256;
  static_assert(LOADS >= 1, "tile too small");

  // Two K/V buffers: tile t+1 is written while tile t is read, so one
  // workgroup barrier per tile suffices.
  __shared__ __attribute__((aligned(16))) uint16_t Ks[NG][2][kBN * K_RS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[NG][2][kBN * V_RS];
  // bf16: V is staged as fp16, each wave's rows scaled by 2^-s (s = 0 unless
  // some |v| >= 2^15; vsc[buffer][wave]), and PV runs as one fp16 MFMA; the
  // softmax folds 2^(s - e_acc) into P and O is kept as acc * 2^e_acc (see
  // prefill_pp_kernel).
  constexpr bool VH = std::is_same<T, BF16>::value;
  __shared__ __attribute__((aligned(16))) int vsc[NG][2][4];

  // ---- work item: longest query blocks first; heads sharing a KV head
  // ---- land on the same XCD (consecutive ids go to consecutive XCDs).
  // Query blocks are counted from each sequence's last row (block jb holds
  // rows [q_len - 128 (jb + 1), q_len - 128 jb)): a partly empty block is a
  // sequence's first, with the shortest causal chain.
  const int per = p.B * p.H;
  const int jb = blockIdx.x / per;
  const int rem = blockIdx.x - jb * per;
  const int b = rem / p.H;
  const int j = rem - b * p.H;
  const int kvh = j % p.Hkv;
  const int h = kvh * p.group + j / p.Hkv;

  const int q_start = p.cu_q[b];
  const int q_len = p.cu_q[b + 1] - q_start;
  constexpr bool PAGED = PG != 0;
  const int k_start = PAGED ? 0 : p.cu_k[b];
  const int kv_len = PAGED ? min(max(p.lens[b], 0), p.max_pages << p.pshift) : p.cu_k[b + 1] - k_start;
  if (jb * kBM >= q_len) return;  // uniform over the workgroup
  const int r_end = q_len - jb * kBM;  // one past the block's last row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int grp = NG > 1 ? __builtin_amdgcn_readfirstlane(tid >> 8) : 0;  // key-tile group
  const int gt = tid & 255;                                               // thread in the group
  const int w = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);           // wave in the group
  const int g = lane >> 5;   // k-group of the MFMA operands
  const int li = lane & 31;  // query column of this lane
  const int shift = kv_len - q_len;
  const int row0 = r_end - kBM + w * 32;  // first query row of this wave (< 0: not stored)
  const int my_row = max(row0 + li, 0);   // rows below 0 compute as row 0
  const float c = p.scale_log2;

  // Q^T operand (B of S^T = K Q^T): lane holds Q[my_row][16 ks + 8 g + 0..7].
  u32x4 qf[KS];
  {
    const uint8_t* qp = p.q + 2 * ((int64_t)(q_start + my_row) * p.q_st + (int64_t)h * p.q_sh + 8 * g);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = (*reinterpret_cast<const u32x4*>(qp + 32 * ks) & p.q_and) ^ p.q_xor;
  }
  // Retire the Q loads here: otherwise the compiler's wait-count tracking
  // keeps treating qf as in flight inside the tile loop and makes every
  // S^T MFMA wait for the K/V prefetch issued just before it.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt untouched

  int hi = kv_len;
  if (CAUSAL) hi = min(kv_len, r_end + shift);
  const int n_all = hi > 0 ? (hi + kBN - 1) / kBN : 0;
  // Steps per group (the same for every group, so barriers pair up); step i
  // of group g is tile g + NG i.  With NG = 2 and n_all odd, group 1's last
  // tile lies past the keys: its loads read zeros or clamped rows and every
  // score is masked.
  const int n_tiles = (n_all + NG - 1) / NG;
  auto gtile = [&](int i) { return grp + NG * i; };

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  float m_run = -INFINITY;  // scaled (log2) units
  float l_run = 0.f;
  int e_acc = 0;  // bf16: O = acc * 2^e_acc

  // K/V prefetch through buffer loads: the sequence's first row (this KV
  // head) is the scalar base and each lane keeps a 32-bit byte offset, so a
  // tile's addresses cost one add per load (no 64-bit vector arithmetic).
  // (Measured: this beats moving the per-load row offset into the scalar
  // descriptor base, whose extra SALU issue slots cost more than the add.)
  const uint8_t* kseq = p.k + 2 * ((int64_t)k_start * p.k_st + (int64_t)kvh * p.k_sh);
  const uint8_t* vseq = p.v + 2 * ((int64_t)k_start * p.v_st + (int64_t)kvh * p.v_sh);
  // Record sizes end at the last row's final byte; loads past them read 0.
  const int k_rec = (int)min((int64_t)max(kv_len - 1, 0) * p.k_st * 2 + 2 * D, (int64_t)0x7fffffff);
  const int v_rec = (int)min((int64_t)max(kv_len - 1, 0) * p.v_st * 2 + 2 * D, (int64_t)0x7fffffff);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kseq, (short)0, k_rec, kBufFlags);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vseq, (short)0, v_rec, kBufFlags);
  const int kst2 = 2 * (int)p.k_st;
  const int vst2 = 2 * (int)p.v_st;
  // Per-lane byte offset of this lane's first chunk; load u adds
  // u * (256 / CPR) rows.  Rows at or past kv_len fall outside the buffer
  // record and read as zero (their scores are masked), so no clamp is needed.
  const int koff0 = (int)__umul24(gt / CPR, kst2) + 16 * (gt % CPR);
  const int voff0 = (int)__umul24(gt / CPR, vst2) + 16 * (gt % CPR);
  constexpr int kRowsPerLoad = 256 / CPR;
  u32x4 kreg[LOADS], vreg[LOADS];
  // Paged streams: the same lane -> (row, chunk) mapping.  PG 1: page id per
  // lane and load; PG 2: page id per load (wave-uniform).
  using Rows = std::conditional_t<PG >= 2, PagedRowsU<LOADS, kRowsPerLoad, PG == 3>, PagedRows<LOADS, kRowsPerLoad>>;
  Rows kpr, vpr;
  if constexpr (PAGED) {
    const int32_t* pt_row = p.pt + (int64_t)b * p.pt_sb;
    kpr.base = p.k + 2 * (int64_t)kvh * p.k_sh;
    vpr.base = p.v + 2 * (int64_t)kvh * p.v_sh;
    kpr.sp2 = 2 * p.k_sp;
    vpr.sp2 = 2 * p.v_sp;
    kpr.st2 = 2 * p.k_st;
    vpr.st2 = 2 * p.v_st;
    kpr.pt_row = vpr.pt_row = pt_row;
    kpr.pshift = vpr.pshift = p.pshift;
    kpr.pmask = vpr.pmask = (1 << p.pshift) - 1;
    kpr.page_last = vpr.page_last = p.num_pages - 1;
    kpr.row0 = vpr.row0 = gt / CPR;
    kpr.tstep = vpr.tstep = NG;
    if constexpr (PG >= 2) {
      kpr.kv_len = vpr.kv_len = kv_len;
      kpr.last_idx = vpr.last_idx = max(kv_len - 1, 0) >> p.pshift;
      kpr.lane_off = (uint32_t)((gt / CPR) * 2 * p.k_st + 16 * (gt % CPR));
      vpr.lane_off = (uint32_t)((gt / CPR) * 2 * p.v_st + 16 * (gt % CPR));
      kpr.cur = vpr.cur = 0;
      kpr.init_pool(p.num_pages);
      vpr.init_pool(p.num_pages);
    } else {
      kpr.kv_last = vpr.kv_last = max(kv_len - 1, 0);
      kpr.col = vpr.col = 16 * (gt % CPR);
    }
    if (n_tiles > 0) {
      kpr.fetch_ids(gtile(0));
      vpr.fetch_ids(gtile(0));
    }
  }
  auto gload_k = [&](int step) {
    const int tile = gtile(step);
    if constexpr (PAGED) {
      kpr.load(tile, kreg);
    } else {
      const int base = koff0 + tile * kBN * kst2;
#pragma unroll
      for (int u = 0; u < LOADS; ++u)
        kreg[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                krs, base + u * kRowsPerLoad * kst2, 0, 0));
    }
  };
  auto gload_v = [&](int step) {
    const int tile = gtile(step);
    if constexpr (PAGED) {
      vpr.load(tile, vreg);
    } else {
      const int base = voff0 + tile * kBN * vst2;
#pragma unroll
      for (int u = 0; u < LOADS; ++u)
        vreg[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                vrs, base + u * kRowsPerLoad * vst2, 0, 0));
    }
  };
  auto lstore_k = [&](int buf) {
    if constexpr (PG >= 2) kpr.mask_tail(kreg);
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int cid = gt + 256 * u;
      *reinterpret_cast<u32x4*>(&Ks[grp][buf][(cid / CPR) * K_RS + 8 * (cid % CPR)]) = kreg[u];
    }
  };
  // bf16: vreg is converted (convert_v) as soon as the step that loaded it
  // has issued its MFMAs, not after the next barrier, so the V loads of the
  // following tile are not delayed behind the conversion; v_s carries the
  // scale to lstore_v.
  int v_s = 0;
  auto convert_v = [&]() {
    if constexpr (VH) {
      if constexpr (PG >= 2) vpr.mask_tail(vreg);
      v_s = bf16_to_f16_scaled<LOADS>(vreg);
    }
  };
  auto lstore_v = [&](int buf) {
    if constexpr (VH) {
      if (lane == 0) vsc[grp][buf][w] = v_s;
    } else if constexpr (PG >= 2) {
      vpr.mask_tail(vreg);
    }
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int cid = gt + 256 * u;
      *reinterpret_cast<u32x4*>(&Vs[grp][buf][(cid / CPR) * V_RS + 8 * (cid % CPR)]) = vreg[u];
    }
  };

  // S^T = K Q^T for the two 32-key blocks of the K tile in Ks[buf].
  auto qk = [&](int buf, f32x16* s) {
    const uint16_t* Kb = Ks[grp][buf];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[jb][r] = 0.f;
    // The two 32-key blocks are independent accumulator chains; alternating
    // them keeps dependent MFMAs apart.
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&Kb[(jb * 32 + li) * K_RS + 16 * ks + 8 * g]);
        s[jb] = Mfma<T>::mma(a, qf[ks], s[jb]);
      }
  };

  // Lane roles of the transposed V reads (see lds_read_tr16).
  const int tr_c = (lane & 15) >> 2;
  const int tr_j = lane & 3;
  const int tr_G = lane >> 4;
  const int tr_row = 4 * (tr_G >> 1) + tr_c;      // + 32 jb + 16 t (+ 8)
  const int tr_col = 16 * (tr_G & 1) + 4 * tr_j;  // + 32 db

  // Software pipeline (one workgroup barrier per tile).  Iteration t
  // computes S(t+1) on the MFMA pipe while the VALU runs the softmax of
  // S(t), then O += V(t) P(t).  K therefore lives two tiles ahead in LDS and
  // V one tile ahead: iteration t stores K(t+2) into Ks[t%2] and V(t+1) into
  // Vs[(t+1)%2] (both buffers were last read in iteration t-1) and issues
  // the global loads of K(t+3) and V(t+2).
  f32x16 s_cur[2];
  if (n_tiles > 0) {
    gload_k(0);
    gload_v(0);
    lstore_k(0);
    convert_v();
    lstore_v(0);
    if (n_tiles > 1) {
      gload_k(1);
      lstore_k(1);
      gload_v(1);
    }
    if (n_tiles > 2) gload_k(2);
    __syncthreads();
    qk(0, s_cur);
    if (n_tiles > 1) convert_v();  // V(1)
  }
  // One pipeline step.  HAS_NEXT (compile time) is false only for the last
  // tile, so S(t+1), the exponentials and the PV MFMAs of every other tile
  // sit in one basic block that the scheduler can interleave; the rare lazy
  // rescale runs in a branch before that block.
  auto step = [&](int tile, auto has_next_tag) {
    constexpr bool HAS_NEXT = decltype(has_next_tag)::value;
    const int buf = tile & 1;
    __syncthreads();
    if (tile + 2 < n_tiles) {
      lstore_k(buf);
      if (tile + 3 < n_tiles) gload_k(tile + 3);
    }
    if (HAS_NEXT) {
      lstore_v(buf ^ 1);
      if (tile + 2 < n_tiles) gload_v(tile + 2);
    }
    const int n0 = gtile(tile) * kBN;
    const uint16_t* Vb = Vs[grp][buf];

    // ---- scores of tile t: mask, row max ----
    const bool need_mask = (n0 + kBN > kv_len) || (CAUSAL && n0 + kBN - 1 > row0 + shift);
    if (need_mask) {  // wave-uniform: only tiles crossing kv_len or the diagonal
      const int lim = CAUSAL ? min(kv_len - 1, my_row + shift) : kv_len - 1;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = n0 + jb * 32 + (r & 3) + 4 * g + 8 * (r >> 2);
          s_cur[jb][r] = key <= lim ? s_cur[jb][r] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_cur[jb][r]);
    mx = xor32<OpMax>(mx);
    mx *= c;  // exact: rounding is monotonic and c > 0
    // Lazy rescale: m_run moves only when this tile's max exceeds it by kLazy.
    const bool grow = mx > m_run + kLazy;
    if (__any(grow)) {
      const float alpha = grow ? fast_exp2(m_run - mx) : 1.f;
      m_run = grow ? mx : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
    }

    // bf16: exponent offsets of the staging waves' V scales for tile t.
    float off[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    float back[2][2] = {{1.f, 1.f}, {1.f, 1.f}};
    if constexpr (VH) v_scale_offsets<CPR>(vsc[grp][buf], g, e_acc, acc, off, back);

    // ---- S(t+1) on the MFMA pipe, interleaved with P(t) = 2^(s c - m) ----
    f32x16 s_nxt[2];
    if constexpr (HAS_NEXT) qk(buf ^ 1, s_nxt);
    const float cm = c;
    // NG > 1: a row can have seen no key yet (its keys lie in the other
    // group's tiles); m_run is then -inf and every score is -inf, so P = 0.
    const float nm = (NG > 1 && m_run == -INFINITY) ? 0.f : -m_run;
    float lsq[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    u32x4 pf[2][2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const float nmo = VH ? nm + off[t][e2 >> 1] : nm;
          const float x0 = fast_exp2(__builtin_fmaf(s_cur[jb][8 * t + 2 * e2], cm, nmo));
          const float x1 = fast_exp2(__builtin_fmaf(s_cur[jb][8 * t + 2 * e2 + 1], cm, nmo));
          // P^T operand: k-step t of key block jb uses accumulator regs 8t..8t+7.
          pf[jb][t][e2] = Pair<F16>::pack(x0, x1);
          // fp32 adds (v_dot2 would stall the other wave's MFMAs); the first
          // pair of each partial sum is assigned, not added to 0.
          if (jb == 0 && (e2 & 1) == 0) lsq[t][e2 >> 1] = x0 + x1;
          else lsq[t][e2 >> 1] += x0 + x1;
        }
    l_run += (lsq[0][0] * back[0][0] + lsq[0][1] * back[0][1]) + (lsq[1][0] * back[1][0] + lsq[1][1] * back[1][1]);

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int vrow = jb * 32 + 16 * t + tr_row;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const uint16_t* vp = &Vb[vrow * V_RS + 32 * db + tr_col];
          const u32x2 lo = lds_read_tr16(vp);
          const u32x2 hi2 = lds_read_tr16(vp + 8 * V_RS);
          const u32x4 a = {lo[0], lo[1], hi2[0], hi2[1]};
          acc[db] = Mfma<F16>::mma(a, pf[jb][t], acc[db]);  // fp16 V and P (bf16: scaled V)
        }
      }
    if constexpr (HAS_NEXT) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) s_cur[jb] = s_nxt[jb];
      if (tile + 2 < n_tiles) convert_v();  // V(t+2), stored by the next step
    }
  };
  for (int tile = 0; tile + 1 < n_tiles; ++tile) step(tile, std::true_type{});
  if (n_tiles > 0) step(n_tiles - 1, std::false_type{});

  if constexpr (NG > 1) {
    // Group 1 hands (O, m, l, e) to the wave of group 0 that owns the same
    // rows, lane for lane, through the tile buffers; group 0 merges.
    constexpr int NV = DB * 16 + 3;
    static_assert(sizeof(Ks) >= 4 * NV * 64 * sizeof(float), "merge buffer");
    float* xch = reinterpret_cast<float*>(&Ks[0][0][0]) + (w * NV) * 64 + lane;  // value e at xch[64 e]
    __syncthreads();  // every wave is done with the tiles
    if (grp == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) xch[64 * (16 * db + r)] = acc[db][r];
      xch[64 * (16 * DB)] = m_run;
      xch[64 * (16 * DB + 1)] = l_run;
      xch[64 * (16 * DB + 2)] = as_f32((u32)e_acc);
    }
    __syncthreads();
    if (grp == 1) return;
    const float m1 = xch[64 * (16 * DB)];
    const float l1 = xch[64 * (16 * DB + 1)];
    const float mm = fmaxf(m_run, m1);
    const float a0 = m_run == -INFINITY ? 0.f : fast_exp2(m_run - mm);
    const float a1 = m1 == -INFINITY ? 0.f : fast_exp2(m1 - mm);
    l_run = l_run * a0 + l1 * a1;  // l is kept unscaled; only O carries 2^e_acc
    float o0 = a0, o1 = a1;
    if constexpr (VH) {
      const int e1 = __builtin_amdgcn_readfirstlane((int)as_u32(xch[64 * (16 * DB + 2)]));
      const int ee = max(e_acc, e1);
      o0 *= as_f32((u32)(127 + e_acc - ee) << 23);
      o1 *= as_f32((u32)(127 + e1 - ee) << 23);
      e_acc = ee;
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] = acc[db][r] * o0 + xch[64 * (16 * db + r)] * o1;
  }

  // ---- epilogue: O = O^T / l.  Each wave stages its 32 rows (as T,
  // row-major) in a wave-private LDS area and stores them row by row, 16
  // contiguous bytes per lane, so an output row leaves in whole cache lines
  // (writing O^T directly puts 8-byte pieces of 32 rows in every store).
  static_assert(sizeof(Vs[0]) >= 4 * kOutStage<D> * sizeof(uint16_t), "output staging");
  if constexpr (NG == 1) __syncthreads();  // every wave is done with the V tiles
  write_rows_via_lds<T, D, DB>(&Vs[0][0][0] + w * kOutStage<D>, li, g, lane, acc, l_run, e_acc, VH, p, q_start,
                               q_len, h, row0);
}


// ---------------------------------------------------------------------------
// Ping-pong variant for grids that fill the chip: 8 waves = 2 groups of 4,
// 256 query rows per workgroup (32 per wave).  Waves w and w + 4 share a
// SIMD and run opposite phases, separated by one workgroup barrier per
// half-step ("slot"):
//   MFMA phase of step t:  S(t+1) = K(t+1) Q^T  and  O += V(t) P(t)
//   VALU phase of step t:  softmax of S(t) -> P(t) (mask, max, lazy rescale,
//                          exponentials), plus this group's staging duty
// Group A (waves 0-3) runs MFMA(t) in slot 2t+2 and VALU(t) in slot 2t+1;
// group B (waves 4-7) one slot later.  So while one wave of a SIMD keeps the
// matrix core busy, the other does its softmax.  Group A stages K tiles
// (stores K(t+1) into Ks[(t+1)&1] in slot 2t+1), group B stages V tiles
// (stores V(t) into Vs[t&1] in slot 2t); each buffer's previous tile was
// last read two slots earlier and the new one is first read one slot later.
// ---------------------------------------------------------------------------
constexpr int kPBM = 256;

// Scheduling groups of one MFMA phase of NE operand entries: the first NS
// entries (S^T blocks) take one LDS read each and feed one MFMA; the rest
// (PV blocks) take two transposed reads each and feed MPP MFMAs.  The reads of
// entry e + LOOK are issued right after the MFMA(s) of entry e.
template <int E, int LOOK, int NE, int NS>
struct MfmaPhaseReads {
  static __device__ __forceinline__ void apply() {
    if constexpr (E < LOOK && E < NE) {
      __builtin_amdgcn_sched_group_barrier(0x100, E < NS ? 1 : 2, 0);
      MfmaPhaseReads<E + 1, LOOK, NE, NS>::apply();
    }
  }
};
template <int E, int NE, int NS, int MPP, int LOOK>
struct MfmaPhaseOrder {
  static __device__ __forceinline__ void apply() {
    if constexpr (E == 0) MfmaPhaseReads<0, LOOK, NE, NS>::apply();
    if constexpr (E < NE) {
      __builtin_amdgcn_sched_group_barrier(0x008, E < NS ? 1 : MPP, 0);
      if constexpr (E + LOOK < NE) __builtin_amdgcn_sched_group_barrier(0x100, (E + LOOK) < NS ? 1 : 2, 0);
      MfmaPhaseOrder<E + 1, NE, NS, MPP, LOOK>::apply();
    }
  }
};

template <typename T, int D, bool CAUSAL, int PG, bool VPRE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_pp_kernel(const PrefillParams p) {
  constexpr int KS = D / 16;
  constexpr int DB = D / 32;
  constexpr int K_RS = D + 8;
  constexpr int V_RS = D + 32;
  constexpr int CPR = D / 8;
  constexpr int LOADS = kBN * CPR / 256;  // one 256-thread group stages a whole tile
  constexpr int kRowsPerLoad = 256 / CPR;
  static_assert(LOADS >= 1, "tile too small");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBN * K_RS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kBN * V_RS];
  // bf16: V tiles are staged as fp16 so that PV runs as one fp16 MFMA with P
  // rounded to fp16 (relative error 2^-11, as on the fp16 path) instead of
  // two bf16 MFMAs with P split into hi + lo parts.  Each staging wave scales
  // its rows by 2^-s (s = 0 unless some |v| >= 2^15), which keeps them inside
  // fp16's range and exact apart from fp16 subnormals (absolute error
  // <= 2^-25 * 2^s); vsc[buffer][wave] holds s.  The softmax folds
  // 2^(s - e_acc) into P's exponent, where O is kept as acc * 2^e_acc.
  constexpr bool VH = std::is_same<T, BF16>::value;
  // VPRE: V arrives as fp16 already, scaled by one power of two per
  // (sequence, KV head) (bf16v_to_f16_kernel), so staging is a plain copy and
  // every wave's scale is that one.
  static_assert(!VPRE || (VH && PG == 0), "V pre-conversion is for packed bf16 prefill");
  __shared__ __attribute__((aligned(16))) int vsc[2][4];

  // Query blocks are counted from each sequence's last row (block jb holds
  // rows [q_len - 256 (jb + 1), q_len - 256 jb)), so a sequence's partly
  // empty block is its first, whose causal chain is the shortest; the grid
  // runs jb = 0 (every sequence's longest chain) first.
  const int per = p.B * p.H;
  const int jb = blockIdx.x / per;
  const int rem = blockIdx.x - jb * per;
  const int b = rem / p.H;
  const int j = rem - b * p.H;
  const int kvh = j % p.Hkv;
  const int h = kvh * p.group + j / p.Hkv;

  const int q_start = p.cu_q[b];
  const int q_len = p.cu_q[b + 1] - q_start;
  constexpr bool PAGED = PG != 0;
  const int k_start = PAGED ? 0 : p.cu_k[b];
  const int kv_len = PAGED ? min(max(p.lens[b], 0), p.max_pages << p.pshift) : p.cu_k[b + 1] - k_start;
  if (jb * kPBM >= q_len) return;  // uniform over the workgroup
  const int r_end = q_len - jb * kPBM;  // one past the block's last row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;     // 0: group A (stages K), 1: group B (stages V)
  const int gt = tid & 255;   // thread index inside the group
  const int g = lane >> 5;
  const int li = lane & 31;
  const int shift = kv_len - q_len;
  // The wave's first row; negative in a sequence's first block when q_len is
  // not a multiple of 256.  Rows below 0 compute as row 0 (my_row) and are
  // not stored.
  const int row0 = r_end - kPBM + w * 32;
  const int my_row = max(row0 + li, 0);
  const float c = p.scale_log2;

  u32x4 qf[KS];
  {
    const int qr = my_row;
    const uint8_t* qp = p.q + 2 * ((int64_t)(q_start + qr) * p.q_st + (int64_t)h * p.q_sh + 8 * g);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = (*reinterpret_cast<const u32x4*>(qp + 32 * ks) & p.q_and) ^ p.q_xor;
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): retire the Q loads before the loop

  int hi = kv_len;
  if (CAUSAL) hi = min(kv_len, r_end + shift);
  const int n_tiles = hi > 0 ? (hi + kBN - 1) / kBN : 0;

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

  // Staging: group A streams K tiles, group B V tiles, through buffer loads
  // (scalar per-sequence base; rows past kv_len read as zero).
  const int st = grp ? (int)p.v_st : (int)p.k_st;
  const int st2 = 2 * st;
  const int64_t sh = grp ? p.v_sh : p.k_sh;
  const uint8_t* seq = (grp ? p.v : p.k) + 2 * ((int64_t)k_start * st + (int64_t)kvh * sh);
  const int rec = (int)min((int64_t)max(kv_len - 1, 0) * st2 + 2 * D, (int64_t)0x7fffffff);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)seq, (short)0, rec, kBufFlags);
  const int off0 = (int)__umul24(gt / CPR, st2) + 16 * (gt % CPR);
  const int lds_rs = grp ? V_RS : K_RS;
  uint16_t* const lds0 = grp ? &Vs[0][0] : &Ks[0][0];
  const int lds_buf = grp ? kBN * V_RS : kBN * K_RS;
  const int lds_off = (gt / CPR) * lds_rs + 8 * (gt % CPR);
  const int vpre_sw = VPRE ? p.v_head_scale[b * p.Hkv + kvh] : 0;
  u32x4 stage[LOADS];
  // PAGED only: this group's K or V stream (PG 1 per-lane page ids, PG 2
  // wave-uniform ones).
  std::conditional_t<PG >= 2, PagedRowsU<LOADS, kRowsPerLoad, PG == 3>, PagedRows<LOADS, kRowsPerLoad>> pr;
  if constexpr (PAGED) {
    pr.base = (grp ? p.v : p.k) + 2 * (int64_t)kvh * sh;
    pr.pt_row = p.pt + (int64_t)b * p.pt_sb;
    pr.sp2 = 2 * (grp ? p.v_sp : p.k_sp);
    pr.st2 = st2;
    pr.pshift = p.pshift;
    pr.pmask = (1 << p.pshift) - 1;
    pr.page_last = p.num_pages - 1;
    pr.row0 = gt / CPR;
    if constexpr (PG >= 2) {
      pr.kv_len = kv_len;
      pr.last_idx = max(kv_len - 1, 0) >> p.pshift;
      pr.lane_off = (uint32_t)((gt / CPR) * st2 + 16 * (gt % CPR));
      pr.cur = 0;
      pr.init_pool(p.num_pages);
    } else {
      pr.kv_last = max(kv_len - 1, 0);
      pr.col = 16 * (gt % CPR);
    }
    if (n_tiles > 0) pr.fetch_ids(0);
  }
  auto gload = [&](int tile) {
    if constexpr (PAGED) {
      pr.load(tile, stage);
    } else {
      const int base = off0 + tile * kBN * st2;
#pragma unroll
      for (int u = 0; u < LOADS; ++u)
        stage[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rs, base + u * kRowsPerLoad * st2, 0, 0));
    }
  };
  auto lstore = [&](int buf) {
    if constexpr (PG >= 2) pr.mask_tail(stage);
    if constexpr (VPRE) {
      if (grp == 1 && lane == 0) vsc[buf][w - 4] = vpre_sw;
    } else if constexpr (VH) {
      if (grp == 1) {
        const int sw = bf16_to_f16_scaled<LOADS>(stage);
        if (lane == 0) vsc[buf][w - 4] = sw;
      }
    }
    uint16_t* dst = lds0 + buf * lds_buf + lds_off;
#pragma unroll
    for (int u = 0; u < LOADS; ++u)
      *reinterpret_cast<u32x4*>(dst + u * kRowsPerLoad * lds_rs) = stage[u];
  };

  const int tr_c = (lane & 15) >> 2;
  const int tr_j = lane & 3;
  const int tr_G = lane >> 4;
  const int tr_row = 4 * (tr_G >> 1) + tr_c;
  const int tr_col = 16 * (tr_G & 1) + 4 * tr_j;

  f32x16 s[2];
  u32x4 pf[2][2];
  int e_acc = 0;  // bf16: O = acc * 2^e_acc

  // S(t) = K(t) Q^T into s.
  auto qk = [&](int t) {
    const uint16_t* Kb = Ks[t & 1];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[jb][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&Kb[(jb * 32 + li) * K_RS + 16 * ks + 8 * g]);
        s[jb] = Mfma<T>::mma(a, qf[ks], s[jb]);
      }
  };
  // O += V(t) P(t).
  auto pv = [&](int t) {
    const uint16_t* Vb = Vs[t & 1];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int vrow = jb * 32 + 16 * tt + tr_row;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const uint16_t* vp = &Vb[vrow * V_RS + 32 * db + tr_col];
          const u32x2 lo = lds_read_tr16(vp);
          const u32x2 hi2 = lds_read_tr16(vp + 8 * V_RS);
          const u32x4 a = {lo[0], lo[1], hi2[0], hi2[1]};
          acc[db] = Mfma<F16>::mma(a, pf[jb][tt], acc[db]);  // fp16 V and P (bf16: scaled V)
        }
      }
  };
  // Staging duty of step t (group A: K(t+1), group B: V(t+1)), then fetch t+2.
  auto stage_step = [&](int t) {
    if (t + 1 < n_tiles) {
      lstore((t + 1) & 1);
      if (t + 2 < n_tiles) gload(t + 2);
    }
  };
  // Softmax of S(t) -> P(t) (mask, max, lazy rescale, exponentials).
  auto softmax = [&](int t) {
    const int n0 = t * kBN;
    const bool need_mask = (n0 + kBN > kv_len) || (CAUSAL && n0 + kBN - 1 > row0 + shift);
    if (need_mask) {
      const int lim = CAUSAL ? min(kv_len - 1, my_row + shift) : kv_len - 1;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = n0 + jb * 32 + (r & 3) + 4 * g + 8 * (r >> 2);
          s[jb][r] = key <= lim ? s[jb][r] : -INFINITY;
        }
    }
    // P(t) = 2^(s c - m_run) against the running max, without a row max:
    // the exact path (row max, lazy rescale, recompute) runs only on the
    // first tile or when some lane's partial row sum exceeds 2^kLazyPP --
    // which every p > 2^kLazyPP forces.  P and the fp32 sums hold values up
    // to 2^kLazyPP exactly as well as values up to 1.
    const float cm = c;
    // bf16: element (tt, e2) of this lane holds a key staged by wave
    // ((4g + 8(2tt + e2/2)) mod kRowsPerLoad) / (64 / CPR) of group B; its
    // P is computed as 2^(s c - m + o) with o = s_wave - e_acc <= 0, and its
    // partial row sum is scaled back by 2^-o.
    float off[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    float back[2][2] = {{1.f, 1.f}, {1.f, 1.f}};
    if constexpr (VH) v_scale_offsets<CPR>(vsc[t & 1], g, e_acc, acc, off, back);
    auto compute_p = [&]() -> float {
      const float nm = -m_run;
      float lsq[2][2] = {{0.f, 0.f}, {0.f, 0.f}};  // four partial row sums
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const float nmo = VH ? nm + off[tt][e2 >> 1] : nm;
            const float x0 = fast_exp2(__builtin_fmaf(s[jb][8 * tt + 2 * e2], cm, nmo));
            const float x1 = fast_exp2(__builtin_fmaf(s[jb][8 * tt + 2 * e2 + 1], cm, nmo));
            pf[jb][tt][e2] = Pair<F16>::pack(x0, x1);
            // fp32 adds, not v_dot2: a dot2 on one wave stalls the other
            // wave's MFMAs (measured on gfx950), undoing the ping-pong overlap.
            // (the first pair of each partial sum is assigned, not added to 0)
            if constexpr (VH) {
              if (jb == 0 && (e2 & 1) == 0) lsq[tt][e2 >> 1] = x0 + x1;
              else lsq[tt][e2 >> 1] += x0 + x1;
            } else {
              if (e2 == 0) lsq[jb][tt] = x0 + x1;
              else lsq[jb][tt] += x0 + x1;
            }
          }
      if constexpr (VH)
        return (lsq[0][0] * back[0][0] + lsq[0][1] * back[0][1]) + (lsq[1][0] * back[1][0] + lsq[1][1] * back[1][1]);
      return (lsq[0][0] + lsq[0][1]) + (lsq[1][0] + lsq[1][1]);
    };
    float ls = 0.f;
    bool exact = t == 0;
    if (!exact) {
      ls = compute_p();
      exact = __any(!(ls <= kLazyPPSum));  // also catches inf / NaN sums
    }
    if (exact) {
      float mx = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[jb][r]);
      mx = xor32<OpMax>(mx);
      mx *= c;
      const bool grow = mx > m_run + kLazyPP;
      if (__any(grow)) {
        const float alpha = grow ? fast_exp2(m_run - mx) : 1.f;
        m_run = grow ? mx : m_run;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
      }
      ls = compute_p();
    }
    l_run += ls;
  };

  // Prologue: K(0) to LDS (group A); K(1) (A) / V(0) (B) into registers.
  // Every wave then passes 2 * n_tiles + 2 barriers; group B runs one slot
  // behind group A, so the two waves of each SIMD are in opposite phases.
  if (n_tiles > 0) {
    gload(0);
    if (grp == 0) {
      lstore(0);
      if (n_tiles > 1) gload(1);
    }
    if (grp == 1) {
      __syncthreads();
      stage_step(-1);  // V(0) -> Vs[0], fetch V(1)
    }
    __syncthreads();
    qk(0);
    __syncthreads();
    stage_step(0);
    softmax(0);
    // Causal: tiles past this wave's last visible key are fully masked for
    // it; from tile nv on the wave only stages tiles and keeps the barrier
    // count (two per tile) of the rest of the workgroup.  A wave whose rows
    // all lie before the sequence's first query (the first block of a
    // sequence whose length is not a multiple of 256) stops after tile 0:
    // nothing it computes is stored.
    const int nv = row0 + 32 <= 0 ? 1 : CAUSAL ? min(n_tiles, (row0 + 31 + shift) / kBN + 1) : n_tiles;
    for (int t = 1; t < nv; ++t) {
      // sched_barrier keeps every instruction inside its phase (the compiler
      // would otherwise move MFMAs across the workgroup barrier); the MFMA
      // phase runs at raised priority so its wave wins issue contention, and
      // its LDS operand reads run 4 MFMAs ahead of their use.
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(2);
      qk(t);
      pv(t - 1);
      MfmaPhaseOrder<0, 2 * KS + 4 * DB, 2 * KS, 1, 4>::apply();
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      stage_step(t);
      softmax(t);
    }
    __syncthreads();
    pv(nv - 1);
    for (int t = nv; t < n_tiles; ++t) {
      __syncthreads();
      stage_step(t);
      __syncthreads();
    }
    if (grp == 0) __syncthreads();
  }

  // Epilogue: waves 0-3 stage their output rows in the K buffers, waves 4-7
  // in the V buffers, once every wave is done with the tiles.
  static_assert(sizeof(Ks) >= 4 * kOutStage<D> * sizeof(uint16_t), "output staging");
  static_assert(sizeof(Vs) >= 4 * kOutStage<D> * sizeof(uint16_t), "output staging");
  __syncthreads();
  write_rows_via_lds<T, D, DB>((w < 4 ? &Ks[0][0] : &Vs[0][0]) + (w & 3) * kOutStage<D>, li, g, lane, acc, l_run,
                               e_acc, VH, p, q_start, q_len, h, row0);
}

// ---------------------------------------------------------------------------
// bf16 V conversion ahead of the ping-pong kernel (VPRE).  The kernel's PV
// product is one fp16 MFMA with P rounded to fp16; bf16 V must therefore be
// staged as fp16.  Converting it inside the kernel costs each group-B wave
// ~80 VALU instructions per tile; converting it once beforehand costs one
// read and one write of V.  One power of two per (sequence, KV head) keeps
// every value inside fp16's range: 2^-s with s = 0 unless some finite |v| of
// that sequence and head is >= 2^15 (then s = its largest exponent - 14).
// Values are exact apart from fp16 subnormals (absolute error <= 2^-25 *
// 2^s), as in the in-kernel form, and a sequence's scale depends on its own
// rows only, so one sequence's magnitudes never reach another's results.
// inf and NaN (exponent field 0xff) stay out of the maximum and convert to
// fp16 inf and NaN.
//
// The pre-pass walks each sequence in 64-row tiles that start at the
// sequence's first row.  Tile t of sequence b records its maximum in slot
// b + floor(cu_k[b] / 64) + t of its head's row of `tilemax`: consecutive
// sequences never share a slot, and every slot is below nblk + B (nblk =
// ceil(total_k / 64)).
// ---------------------------------------------------------------------------
constexpr int kVpreRows = 64;  // V rows per pre-pass tile

// Rows [r0, r1) of sequence b (clamped into [0, total_k)) and its tile count.
struct VpreSeq {
  int r0, r1, ntiles, slot0;
};
__device__ __forceinline__ VpreSeq vpre_seq(const int32_t* __restrict__ cu_k, int b, int total_k, int nslot) {
  VpreSeq s;
  s.r0 = min(max(cu_k[b], 0), total_k);
  s.r1 = min(max(cu_k[b + 1], s.r0), total_k);
  s.ntiles = (s.r1 - s.r0 + kVpreRows - 1) / kVpreRows;
  s.slot0 = b + s.r0 / kVpreRows;
  s.ntiles = min(s.ntiles, max(nslot - s.slot0, 0));  // in range for any cu_k
  return s;
}

// Largest finite bf16 exponent field of |v| over tile t of sequence b, KV
// head h -> tilemax[h * nslot + slot].  Grid (x, Hkv, B); workgroup x takes
// tiles x, x + gridDim.x, ...
template <int D>
__global__ __launch_bounds__(256) void bf16v_expmax_kernel(const uint16_t* __restrict__ v, int64_t v_st,
                                                           int64_t v_sh, const int32_t* __restrict__ cu_k,
                                                           int total_k, int nslot,
                                                           int32_t* __restrict__ tilemax) {
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const VpreSeq sq = vpre_seq(cu_k, b, total_k, nslot);
  __shared__ u32 red[4];
  for (int t = blockIdx.x; t < sq.ntiles; t += gridDim.x) {
    u32 em = 0;
    for (int c = threadIdx.x; c < kVpreRows * CPR; c += 256) {
      const int row = sq.r0 + t * kVpreRows + c / CPR;
      if (row < sq.r1) {
        const u32x4 x =
            *reinterpret_cast<const u32x4*>(v + (int64_t)row * v_st + (int64_t)h * v_sh + 8 * (c % CPR));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const u32 lo = x[e] & 0x7f80u, hi = (x[e] >> 16) & 0x7f80u;
          em = max(em, max(lo == 0x7f80u ? 0u : lo, hi == 0x7f80u ? 0u : hi));
        }
      }
    }
    u32 m = em;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, (u32)__shfl_xor((int)m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0)
      tilemax[(int64_t)h * nslot + sq.slot0 + t] = (int32_t)(max(max(red[0], red[1]), max(red[2], red[3])) >> 7);
    __syncthreads();
  }
}

// fp16(v * 2^-s) of the tiles of sequence b, KV head h, into the dense
// [total_k, Hkv, D] array v16, where s is the (b, h) scale taken from that
// sequence's tile maxima; workgroup (0, h, b) records s in
// seq_scale[b * Hkv + h] (0 for a sequence without keys).
template <int D>
__global__ __launch_bounds__(256) void bf16v_to_f16_kernel(const uint16_t* __restrict__ v, int64_t v_st, int64_t v_sh,
                                                           const int32_t* __restrict__ cu_k, int total_k, int Hkv,
                                                           int nslot, const int32_t* __restrict__ tilemax,
                                                           uint16_t* __restrict__ v16,
                                                           int32_t* __restrict__ seq_scale) {
  constexpr int CPR = D / 8;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const VpreSeq sq = vpre_seq(cu_k, b, total_k, nslot);
  int le = 0;
  for (int i = threadIdx.x; i < sq.ntiles; i += 256) le = max(le, tilemax[(int64_t)h * nslot + sq.slot0 + i]);
  __shared__ int red[4];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) le = max(le, __shfl_xor(le, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = le;
  __syncthreads();
  le = max(max(red[0], red[1]), max(red[2], red[3]));
  const int sw = max(0, le - 141);  // 2^(le - 127) >= 2^15 <=> le >= 142; finite le <= 254
  if (blockIdx.x == 0 && threadIdx.x == 0) seq_scale[b * Hkv + h] = sw;
  const float f = as_f32((u32)(127 - sw) << 23);  // 2^-sw, sw <= 113
  for (int t = blockIdx.x; t < sq.ntiles; t += gridDim.x) {
    for (int c = threadIdx.x; c < kVpreRows * CPR; c += 256) {
      const int row = sq.r0 + t * kVpreRows + c / CPR;
      if (row >= sq.r1) continue;
      const u32x4 x = *reinterpret_cast<const u32x4*>(v + (int64_t)row * v_st + (int64_t)h * v_sh + 8 * (c % CPR));
      u32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = Pair<F16>::pack(Pair<BF16>::lo(x[e]) * f, Pair<BF16>::hi(x[e]) * f);
      *reinterpret_cast<u32x4*>(v16 + ((int64_t)row * Hkv + h) * D + 8 * (c % CPR)) = y;
    }
  }
}

}  // namespace fat

// ===========================================================================
// Host side
// ===========================================================================
namespace {

template <typename T, int D, bool CAUSAL, int PG, int NG>
void launch_prefill_c(const fat::PrefillParams& prm, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((fat::prefill_kernel<T, D, CAUSAL, PG, NG>), grid, dim3(256 * NG), 0, stream, prm);
}

template <typename T, int D, bool CAUSAL, int PG, bool VPRE = false>
void launch_prefill_pp_c(const fat::PrefillParams& prm, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((fat::prefill_pp_kernel<T, D, CAUSAL, PG, VPRE>), grid, dim3(512), 0, stream, prm);
}

// Mean query tokens per sequence from which bf16 packed prefill converts V
// to fp16 ahead of the ping-pong kernel (when given the workspace).
constexpr int64_t kVpreMinMeanQ = 2048;

// Kernel families of the prefill launch.
enum PrefillKind { PF_PINGPONG, PF_4WAVE, PF_4WAVE_SPLIT, PF_WIDE };

// Bytes of the fp16 copy of V in the prefill workspace (256-byte aligned).
size_t vpre_bytes_v16(int64_t total_k, int64_t hkv, int64_t d) {
  return (size_t)((total_k * hkv * d * 2 + 255) / 256 * 256);
}

template <typename T, int D, int PG>
int launch_prefill_t(const fat::PrefillParams& prm, bool causal, PrefillKind kind, dim3 grid, hipStream_t stream) {
  if constexpr (D == 256) {  // the 4-wave kernel only (launch_prefill checked kind)
    (void)kind;
    if (causal) launch_prefill_c<T, D, true, PG, 1>(prm, grid, stream);
    else launch_prefill_c<T, D, false, PG, 1>(prm, grid, stream);
    return fat_host::launch_status("prefill_kernel");
  } else {
    if (kind == PF_PINGPONG) {
      if constexpr (std::is_same<T, fat::BF16>::value && PG == 0) {
        if (prm.v_head_scale) {
          if (causal) launch_prefill_pp_c<T, D, true, PG, true>(prm, grid, stream);
          else launch_prefill_pp_c<T, D, false, PG, true>(prm, grid, stream);
          return fat_host::launch_status("prefill_pp_kernel");
        }
      }
      if (causal) launch_prefill_pp_c<T, D, true, PG>(prm, grid, stream);
      else launch_prefill_pp_c<T, D, false, PG>(prm, grid, stream);
      return fat_host::launch_status("prefill_pp_kernel");
    }
    if (kind == PF_4WAVE_SPLIT) {
      if (causal) launch_prefill_c<T, D, true, PG, 2>(prm, grid, stream);
      else launch_prefill_c<T, D, false, PG, 2>(prm, grid, stream);
    } else {
      if (causal) launch_prefill_c<T, D, true, PG, 1>(prm, grid, stream);
      else launch_prefill_c<T, D, false, PG, 1>(prm, grid, stream);
    }
    return fat_host::launch_status("prefill_kernel");
  }
}

template <typename T, int PG>
int launch_prefill_d(const fat::PrefillParams& prm, int D, bool causal, PrefillKind kind, dim3 grid,
                     hipStream_t stream) {
  switch (D) {
    case 128: return launch_prefill_t<T, 128, PG>(prm, causal, kind, grid, stream);
    case 64: return launch_prefill_t<T, 64, PG>(prm, causal, kind, grid, stream);
    case 32: return launch_prefill_t<T, 32, PG>(prm, causal, kind, grid, stream);
    default: return launch_prefill_t<T, 256, PG>(prm, causal, kind, grid, stream);  // 256 (checked)
  }
}

bool valid_prefill_kernel(int kernel) {
  return kernel == FAT_KERNEL_AUTO || kernel == FAT_KERNEL_PREFILL_PINGPONG || kernel == FAT_KERNEL_PREFILL_4WAVE ||
         kernel == FAT_KERNEL_PREFILL_4WAVE_SPLIT || kernel == FAT_KERNEL_PREFILL_WIDE ||
         kernel == FAT_KERNEL_PREFILL_GENERIC;
}

// fp32 and head_dim 16 / 512 have no MFMA prefill kernel: the generic one
// (prefill_generic.hip) takes them; forcing it runs it on any shape.
bool prefill_needs_generic(int dtype, int D) { return dtype == FAT_DTYPE_F32 || D == 16 || D == 512; }

// Whether the bf16 V pre-pass can run for a packed launch (its arrays fit
// fat_prefill_workspace_bytes, and the dense fp16 copy keeps the kernels'
// 32-bit per-sequence offsets); whether it pays is decided by the caller.
bool vpre_fits(int64_t B, int64_t Hkv, int D, int64_t total_k, int64_t max_seqlen_k) {
  if (D == 256 || total_k <= 0) return false;
  if (max_seqlen_k * 2 * Hkv * D >= 0x7fffffffLL || 2 * Hkv * D >= (1 << 24)) return false;
  const int64_t nblk = (total_k + fat::kVpreRows - 1) / fat::kVpreRows;
  return 2 * B <= nblk + 1;
}

// Kernel choice and grid shared by fat_prefill_varlen and fat_prefill_paged.
// A workgroup's time is its chain of 64-key tiles, up to ceil(max_seqlen_k /
// 64) for the longest query block; the launch ends with the longest chain on
// the busiest CU.  The 8-wave ping-pong kernel (256 query rows, one
// workgroup per CU) is the fastest per tile once its grid covers the 256 CUs:
// non-causal grids of at least FAT_PF_PP_MIN_FULL workgroups, causal grids
// (whose blocks differ in length) of more than FAT_PF_PP_MIN_CAUSAL.  Below
// that the 4-wave kernel (128 rows, two workgroups per CU) runs, or its
// 8-wave split form, whose two groups take alternate key tiles of one query
// block and so halve its chain, when the 4-wave grid leaves CUs idle (at most
// FAT_PF_SPLIT_MAX workgroups) and the chain is at least FAT_PF_SPLIT_TILES
// tiles, or, causal, when it has at most 2 FAT_PF_SPLIT_MAX workgroups and
// chains of at least FAT_PF_SPLIT_LONG tiles (the merge then costs less than
// the balance gained).  A non-AUTO `kernel` argument forces one kernel (the
// tests run every kernel on every shape that way).
PrefillKind choose_prefill_kind(int64_t B, int64_t H, int max_seqlen_q, int64_t max_seqlen_k, bool causal,
                                int kernel, int D, int dtype, bool packed, bool vpre_ok, int64_t total_q) {
  const int64_t heads = B * H;
  const int64_t n_pp = (max_seqlen_q + fat::kPBM - 1) / fat::kPBM * heads;
  const int64_t n_4w = (max_seqlen_q + fat::kBM - 1) / fat::kBM * heads;
  const int64_t n_wide = (max_seqlen_q + fat::kWideBM - 1) / fat::kWideBM * heads;
  const int64_t chain = (max_seqlen_k + fat::kBN - 1) / fat::kBN;
  PrefillKind kind = PF_4WAVE;
  if (causal ? n_pp > FAT_PF_PP_MIN_CAUSAL : n_pp >= FAT_PF_PP_MIN_FULL) kind = PF_PINGPONG;
  else if ((n_4w <= FAT_PF_SPLIT_MAX && chain >= FAT_PF_SPLIT_TILES) ||
           (causal && n_4w <= 2 * FAT_PF_SPLIT_MAX && chain >= FAT_PF_SPLIT_LONG))
    kind = PF_4WAVE_SPLIT;
  // The 64-rows-per-wave kernel once its 512-row blocks alone cover the CUs
  // (causal grids: more than that, as for the ping-pong kernel), for packed
  // fp16 at head_dim 128, and bf16 whose V the pre-pass converts, when the
  // sequences average at least FAT_PF_WIDE_MEAN queries: a sequence's partly
  // empty block (its first) costs a 512-row block's chain.  Measured (32/8
  // heads, D128, one box, fp16 causal against the ping-pong kernel): 5 %
  // faster at L8192, 1-3 % on packs of 8 or 16 sequences drawn from
  // [1, 4096] (means 1950-2500), level at 8 x 2048, 7-8 % slower at means
  // near 1000; bf16 and non-causal gain from a mean of 2048.
  if (kind == PF_PINGPONG && packed && D == 128 && (dtype == FAT_DTYPE_F16 || vpre_ok) &&
      (causal ? n_wide > FAT_PF_WIDE_MIN_CAUSAL : n_wide >= FAT_PF_WIDE_MIN_FULL) &&
      total_q >= FAT_PF_WIDE_MEAN * B)
    kind = PF_WIDE;
  if (kernel != FAT_KERNEL_AUTO) {
    kind = kernel == FAT_KERNEL_PREFILL_PINGPONG ? PF_PINGPONG
           : kernel == FAT_KERNEL_PREFILL_4WAVE  ? PF_4WAVE
           : kernel == FAT_KERNEL_PREFILL_WIDE   ? PF_WIDE
                                                 : PF_4WAVE_SPLIT;
  }
  if (D == 256) kind = PF_4WAVE;  // see launch_prefill
  return kind;
}

// Workspace bytes of the bf16 V pre-pass of a packed launch, or 0 when the
// launch converts V in the kernel instead.  The wide kernel needs the
// pre-pass; the ping-pong kernel runs it when the sequences average at
// least kVpreMinMeanQ query tokens (where the copy costs less than it saves:
// the pre-pass reads V twice and writes it once, while the kernel converts
// each V tile once per (query block, query head) that stages it; measured
// (bf16, 32/8 heads, D128): 3-6 % faster from a mean of 2048 query tokens
// per sequence, level at 1024, 1-5 % slower at 512).  vpre_fits bounds the
// rest.  Layout: the fp16 copy [total_k, Hkv, D] (256-byte aligned), tile
// maxima [Hkv, nblk + B], scales [B, Hkv].
size_t vpre_need(PrefillKind kind, int dtype, int64_t B, int64_t Hkv, int D, int64_t total_q, int64_t total_k,
                 int64_t max_seqlen_k) {
  if (dtype != FAT_DTYPE_BF16 || !vpre_fits(B, Hkv, D, total_k, max_seqlen_k)) return 0;
  if (kind != PF_WIDE && !(kind == PF_PINGPONG && total_q >= kVpreMinMeanQ * B)) return 0;
  const int64_t nblk = (total_k + fat::kVpreRows - 1) / fat::kVpreRows;
  return vpre_bytes_v16(total_k, Hkv, D) + (size_t)(Hkv * (nblk + 2 * B)) * sizeof(int32_t);
}

template <int PG>
int launch_prefill(fat::PrefillParams& prm, int max_seqlen_q, int64_t max_seqlen_k, int dtype, int D, bool causal,
                   float softmax_scale, int kernel, const char* who, hipStream_t stream, void* workspace = nullptr,
                   int total_k = 0, int total_q = 0) {
  if (prefill_needs_generic(dtype, D) || kernel == FAT_KERNEL_PREFILL_GENERIC) {
    if (kernel != FAT_KERNEL_AUTO && kernel != FAT_KERNEL_PREFILL_GENERIC) {
      fat_host::set_error("%s: %s runs on the generic prefill kernel only (kernel %d)", who,
                          dtype == FAT_DTYPE_F32 ? "fp32" : "this head_dim", kernel);
      return FAT_E_UNSUPPORTED;
    }
    prm.nqb = (max_seqlen_q + 31) / 32;
    prm.scale_log2 = softmax_scale * fat::kLog2e;
    const int64_t n = (int64_t)prm.nqb * prm.B * prm.H;
    if (n > 0x7fffffff) {
      fat_host::set_error("%s: too many query blocks (%lld)", who, (long long)n);
      return FAT_E_UNSUPPORTED;
    }
    return fat_host::launch_prefill_generic(prm, dtype, D, causal, PG != 0, dim3((unsigned)n), stream);
  }
  const bool vpre_ok = PG == 0 && workspace && vpre_fits(prm.B, prm.Hkv, D, total_k, max_seqlen_k);
  PrefillKind kind = choose_prefill_kind(prm.B, prm.H, max_seqlen_q, max_seqlen_k, causal, kernel, D, dtype,
                                         PG == 0, vpre_ok, total_q);
  if (kind == PF_WIDE && (PG != 0 || D != 128 || (dtype == FAT_DTYPE_BF16 && !vpre_ok))) {
    fat_host::set_error("%s: the wide prefill kernel takes packed head_dim-128 launches (bf16 with the "
                        "workspace of fat_prefill_varlen_workspace_bytes) only", who);
    return FAT_E_UNSUPPORTED;
  }
  // head_dim 256: O and Q alone take 192 registers per lane, so only the
  // 4-wave kernel (one wave per SIMD) runs it; its K/V tiles take 141 KB of
  // LDS, which leaves no room for the split's second group.
  if (D == 256) {
    if (kernel != FAT_KERNEL_AUTO && kernel != FAT_KERNEL_PREFILL_4WAVE) {
      fat_host::set_error("%s: head_dim 256 runs on the 4-wave prefill kernel only (kernel %d)", who, kernel);
      return FAT_E_UNSUPPORTED;
    }
    kind = PF_4WAVE;
  }
  const int bm = kind == PF_WIDE ? fat::kWideBM : kind == PF_PINGPONG ? fat::kPBM : fat::kBM;
  prm.nqb = (max_seqlen_q + bm - 1) / bm;
  // The MFMA kernels take a positive scale: a negative one runs as its
  // magnitude with Q's signs flipped as Q is loaded (exact in fp16/bf16 and
  // through the MFMA sums), a zero one with Q zeroed (every logit 0).
  prm.q_and = ~0u;
  prm.q_xor = 0u;
  prm.scale_log2 = softmax_scale * fat::kLog2e;
  if (softmax_scale < 0.f) {
    prm.q_xor = 0x80008000u;
    prm.scale_log2 = -prm.scale_log2;
  } else if (softmax_scale == 0.f) {
    prm.q_and = 0u;
    prm.scale_log2 = fat::kLog2e;
  }
  const int64_t n = (int64_t)prm.nqb * prm.B * prm.H;
  if (n > 0x7fffffff) {
    fat_host::set_error("%s: too many query blocks (%lld)", who, (long long)n);
    return FAT_E_UNSUPPORTED;
  }
  const dim3 grid((unsigned)n);
  // Packed bf16 on the ping-pong kernel: convert V to fp16 first (vpre_need)
  // when the caller gave the workspace.
  prm.v_head_scale = nullptr;
  if (PG == 0 && workspace && vpre_need(kind, dtype, prm.B, prm.Hkv, D, total_q, total_k, max_seqlen_k) > 0) {
    const int nblk = (total_k + fat::kVpreRows - 1) / fat::kVpreRows;
    const int nslot = nblk + prm.B;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    uint16_t* v16 = reinterpret_cast<uint16_t*>(ws);
    int32_t* tilemax = reinterpret_cast<int32_t*>(ws + vpre_bytes_v16(total_k, prm.Hkv, D));
    int32_t* seq_scale = tilemax + (int64_t)prm.Hkv * nslot;
    // One workgroup per tile of the longest sequence (max_seqlen_k bounds the
    // tile count; a workgroup loops over the tiles beyond gridDim.x anyway).
    const int64_t tiles = (max_seqlen_k + fat::kVpreRows - 1) / fat::kVpreRows;
    const dim3 pgrid((unsigned)std::max<int64_t>(1, std::min<int64_t>(tiles, 65535)), (unsigned)prm.Hkv,
                     (unsigned)prm.B);
    const uint16_t* vsrc = reinterpret_cast<const uint16_t*>(prm.v);
    const int32_t* cuk = prm.cu_k;
    if (D == 128) {
      hipLaunchKernelGGL((fat::bf16v_expmax_kernel<128>), pgrid, dim3(256), 0, stream, vsrc, prm.v_st, prm.v_sh,
                         cuk, total_k, nslot, tilemax);
      hipLaunchKernelGGL((fat::bf16v_to_f16_kernel<128>), pgrid, dim3(256), 0, stream, vsrc, prm.v_st, prm.v_sh,
                         cuk, total_k, prm.Hkv, nslot, tilemax, v16, seq_scale);
    } else if (D == 64) {
      hipLaunchKernelGGL((fat::bf16v_expmax_kernel<64>), pgrid, dim3(256), 0, stream, vsrc, prm.v_st, prm.v_sh,
                         cuk, total_k, nslot, tilemax);
      hipLaunchKernelGGL((fat::bf16v_to_f16_kernel<64>), pgrid, dim3(256), 0, stream, vsrc, prm.v_st, prm.v_sh,
                         cuk, total_k, prm.Hkv, nslot, tilemax, v16, seq_scale);
    } else {
      hipLaunchKernelGGL((fat::bf16v_expmax_kernel<32>), pgrid, dim3(256), 0, stream, vsrc, prm.v_st, prm.v_sh,
                         cuk, total_k, nslot, tilemax);
      hipLaunchKernelGGL((fat::bf16v_to_f16_kernel<32>), pgrid, dim3(256), 0, stream, vsrc, prm.v_st, prm.v_sh,
                         cuk, total_k, prm.Hkv, nslot, tilemax, v16, seq_scale);
    }
    const int rc = fat_host::launch_status("bf16v_to_f16_kernel");
    if (rc != FAT_OK) return rc;
    prm.v = reinterpret_cast<const uint8_t*>(v16);
    prm.v_st = (int64_t)prm.Hkv * D;
    prm.v_sh = D;
    prm.v_head_scale = seq_scale;
  }
  if (kind == PF_WIDE) {
    // Packs of 2-16 sequences run their (query block, sequence) items
    // longest chain first (the kernel ranks them: O(B) per thread, at most
    // 512 items, one per thread).
    const int64_t items = (int64_t)prm.nqb * prm.B;
    prm.rank_items = (prm.B >= 2 && prm.B <= fat::kWideRankMaxSeqs && items <= fat::kWideBM) ? (int)items : 0;
    return fat_host::launch_prefill_wide(prm, dtype == FAT_DTYPE_BF16, causal, grid, stream);
  }
  if (dtype == FAT_DTYPE_F16) return launch_prefill_d<fat::F16, PG>(prm, D, causal, kind, grid, stream);
  return launch_prefill_d<fat::BF16, PG>(prm, D, causal, kind, grid, stream);
}

}  // namespace

extern "C" size_t fat_prefill_workspace_bytes(int32_t total_k, int32_t num_kv_heads, int32_t head_dim) {
  if (total_k <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  const size_t nblk = ((size_t)total_k + fat::kVpreRows - 1) / fat::kVpreRows;
  return vpre_bytes_v16(total_k, num_kv_heads, head_dim) + (2 * nblk + 1) * (size_t)num_kv_heads * sizeof(int32_t);
}

extern "C" size_t fat_prefill_varlen_workspace_bytes(const fat_prefill_args* a) {
  if (!a || a->batch <= 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->total_q <= 0 || a->total_k <= 0 ||
      a->max_seqlen_q <= 0 || a->max_seqlen_k < 0 || !valid_prefill_kernel(a->kernel))
    return 0;
  if (prefill_needs_generic(a->dtype, a->head_dim) || a->kernel == FAT_KERNEL_PREFILL_GENERIC) return 0;
  const bool fits = vpre_fits(a->batch, a->num_kv_heads, a->head_dim, a->total_k, a->max_seqlen_k);
  const PrefillKind kind = choose_prefill_kind(a->batch, a->num_heads, a->max_seqlen_q, a->max_seqlen_k,
                                               a->causal != 0, a->kernel, a->head_dim, a->dtype, true, fits,
                                               a->total_q);
  return vpre_need(kind, a->dtype, a->batch, a->num_kv_heads, a->head_dim, a->total_q, a->total_k,
                   a->max_seqlen_k);
}

extern "C" int fat_prefill_varlen(const fat_prefill_args* a, void* stream_ptr) {
  fat_host::clear_error();
  if (!a) {
    fat_host::set_error("fat_prefill_varlen: args is NULL");
    return FAT_E_INVALID;
  }
  if (!a->q || !a->k || !a->v || !a->cu_seqlens_q || !a->cu_seqlens_k || !a->out) {
    fat_host::set_error("fat_prefill_varlen: a required pointer is NULL");
    return FAT_E_INVALID;
  }
  if (a->batch <= 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->total_q < 0 || a->total_k < 0) {
    fat_host::set_error("fat_prefill_varlen: batch and head counts must be positive");
    return FAT_E_INVALID;
  }
  if (a->num_heads % a->num_kv_heads != 0) {
    fat_host::set_error("fat_prefill_varlen: num_heads %d must be divisible by num_kv_heads %d", a->num_heads,
                        a->num_kv_heads);
    return FAT_E_INVALID;
  }
  if (a->dtype != FAT_DTYPE_F16 && a->dtype != FAT_DTYPE_BF16 && a->dtype != FAT_DTYPE_F32) {
    fat_host::set_error("fat_prefill_varlen: dtype must be fp16, bf16 or fp32");
    return FAT_E_UNSUPPORTED;
  }
  const int64_t esz = a->dtype == FAT_DTYPE_F32 ? 4 : 2;  // bytes per element
  if (!valid_prefill_kernel(a->kernel)) {
    fat_host::set_error("fat_prefill_varlen: kernel must be FAT_KERNEL_AUTO (0), _PREFILL_PINGPONG (1), "
                        "_PREFILL_4WAVE (2), _PREFILL_4WAVE_SPLIT (3), _PREFILL_WIDE (4) or _PREFILL_GENERIC (5), "
                        "got %d", a->kernel);
    return FAT_E_INVALID;
  }
  const int D = a->head_dim;
  if (D < 16 || D > 512 || (D & (D - 1)) != 0) {
    fat_host::set_error("fat_prefill_varlen: head_dim %d unsupported (a power of two from 16 to 512)", D);
    return FAT_E_UNSUPPORTED;
  }
  if (a->max_seqlen_q < 0 || a->max_seqlen_k < 0) {
    fat_host::set_error("fat_prefill_varlen: max_seqlen must be non-negative");
    return FAT_E_INVALID;
  }
  const uintptr_t align16 = (uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->v | (uintptr_t)(esz * a->q_stride_t) |
                            (uintptr_t)(esz * a->q_stride_h) | (uintptr_t)(esz * a->k_stride_t) |
                            (uintptr_t)(esz * a->k_stride_h) | (uintptr_t)(esz * a->v_stride_t) |
                            (uintptr_t)(esz * a->v_stride_h);
  const uintptr_t align8 =
      (uintptr_t)a->out | (uintptr_t)(esz * a->out_stride_t) | (uintptr_t)(esz * a->out_stride_h);
  if ((align16 & 15) || (align8 & 7)) {
    fat_host::set_error("fat_prefill_varlen: q/k/v rows must be 16-byte aligned and out rows 8-byte aligned");
    return FAT_E_INVALID;
  }
  // Per-sequence K/V byte offsets are 32-bit (row * 2 * stride, 24-bit
  // multiply): every kv_len is bounded by max_seqlen_k.
  const int64_t kv_stride = a->k_stride_t > a->v_stride_t ? a->k_stride_t : a->v_stride_t;
  if (kv_stride <= 0 || esz * kv_stride >= (1 << 24) || (int64_t)a->max_seqlen_k * esz * kv_stride >= 0x7fffffffLL) {
    fat_host::set_error("fat_prefill_varlen: max_seqlen_k %d x token stride %lld exceeds the kernel's 32-bit "
                        "per-sequence K/V offsets", a->max_seqlen_k, (long long)kv_stride);
    return FAT_E_UNSUPPORTED;
  }
  if (a->max_seqlen_q == 0 || a->total_q == 0) return FAT_OK;  // nothing to compute

  fat::PrefillParams prm{};
  prm.q = static_cast<const uint8_t*>(a->q);
  prm.k = static_cast<const uint8_t*>(a->k);
  prm.v = static_cast<const uint8_t*>(a->v);
  prm.cu_q = a->cu_seqlens_q;
  prm.cu_k = a->cu_seqlens_k;
  prm.out = static_cast<uint8_t*>(a->out);
  prm.q_st = a->q_stride_t;
  prm.q_sh = a->q_stride_h;
  prm.k_st = a->k_stride_t;
  prm.k_sh = a->k_stride_h;
  prm.v_st = a->v_stride_t;
  prm.v_sh = a->v_stride_h;
  prm.o_st = a->out_stride_t;
  prm.o_sh = a->out_stride_h;
  prm.B = a->batch;
  prm.H = a->num_heads;
  prm.Hkv = a->num_kv_heads;
  prm.group = a->num_heads / a->num_kv_heads;
  if (a->workspace && ((uintptr_t)a->workspace & 255)) {
    fat_host::set_error("fat_prefill_varlen: workspace must be 256-byte aligned");
    return FAT_E_INVALID;
  }
  return launch_prefill<0>(prm, a->max_seqlen_q, a->max_seqlen_k, a->dtype, D, a->causal != 0, a->softmax_scale,
                           a->kernel, "fat_prefill_varlen", static_cast<hipStream_t>(stream_ptr), a->workspace,
                           a->total_k, a->total_q);
}

// Staging plan of a paged launch (prefill_stage.hip): the rows of packed K/V
// copies (batch x max_pages x page_size, the table's capacity) when the
// launch runs on the wide kernel through them, else 0.  Taken when the packed
// launch of the same shape would run the wide kernel (fp16, or bf16 whose
// copied V the pre-pass converts; head_dim 128; sequences averaging
// FAT_PF_WIDE_MEAN queries or more, choose_prefill_kind; fp16 causal
// launches FAT_PF_STAGE_MEAN_F16_CAUSAL unless the wide kernel is asked
// for, since there the wide kernel gains
// least over the paged ping-pong kernel and the copies cost the same), when
// the copies hold at most 4 rows per query (the workspace stays in
// proportion to the launch) and fit the packed kernels' 32-bit offsets.  The
// copies cost one read and one write of the used K/V rows; the wide kernel
// then reads each row once per query block, 16 bytes a lane straight into
// LDS.
#ifndef FAT_PF_STAGE_MEAN_F16_CAUSAL
#define FAT_PF_STAGE_MEAN_F16_CAUSAL 4096
#endif
int64_t paged_stage_rows(const fat_prefill_paged_args* a) {
  if (a->head_dim != 128 || (a->dtype != FAT_DTYPE_F16 && a->dtype != FAT_DTYPE_BF16)) return 0;
  if (a->kernel != FAT_KERNEL_AUTO && a->kernel != FAT_KERNEL_PREFILL_WIDE) return 0;
  if (a->batch <= 0 || a->batch > 65535 || a->total_q <= 0 || a->max_seqlen_q <= 0 || a->num_kv_heads <= 0 ||
      a->num_heads <= 0 || a->max_pages <= 0 || a->page_size <= 0)
    return 0;
  const int64_t cap = (int64_t)a->max_pages * a->page_size;
  const int64_t rows = cap * a->batch;
  if (rows > 4 * (int64_t)a->total_q || rows * a->num_kv_heads * a->head_dim * 2 >= 0x7fffffffLL) return 0;
  const bool fits = vpre_fits(a->batch, a->num_kv_heads, a->head_dim, rows, cap);
  if (a->dtype == FAT_DTYPE_BF16 && !fits) return 0;
  if (a->kernel == FAT_KERNEL_AUTO && a->dtype == FAT_DTYPE_F16 && a->causal &&
      a->total_q < (int64_t)FAT_PF_STAGE_MEAN_F16_CAUSAL * a->batch)
    return 0;
  const PrefillKind kind = choose_prefill_kind(a->batch, a->num_heads, a->max_seqlen_q, cap, a->causal != 0,
                                               a->kernel, a->head_dim, a->dtype, true, fits, a->total_q);
  return kind == PF_WIDE ? rows : 0;
}

// Workspace of a staged paged launch (256-byte aligned parts): cu_k [B + 1],
// the K and V copies [rows, Hkv, D], then the bf16 V pre-pass area.
struct PagedStageLayout {
  size_t k, v, vpre, total;
};
PagedStageLayout paged_stage_layout(const fat_prefill_paged_args* a, int64_t rows) {
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t kv = al((size_t)rows * a->num_kv_heads * a->head_dim * 2);
  PagedStageLayout L;
  L.k = al((size_t)(a->batch + 1) * sizeof(int32_t));
  L.v = L.k + kv;
  L.vpre = L.v + kv;
  L.total = L.vpre + vpre_need(PF_WIDE, a->dtype, a->batch, a->num_kv_heads, a->head_dim, a->total_q, rows,
                               (int64_t)a->max_pages * a->page_size);
  return L;
}

extern "C" size_t fat_prefill_paged_workspace_bytes(const fat_prefill_paged_args* a) {
  if (!a) return 0;
  const int64_t rows = paged_stage_rows(a);
  return rows > 0 ? paged_stage_layout(a, rows).total : 0;
}

extern "C" int fat_prefill_paged(const fat_prefill_paged_args* a, void* stream_ptr) {
  fat_host::clear_error();
  if (!a) {
    fat_host::set_error("fat_prefill_paged: args is NULL");
    return FAT_E_INVALID;
  }
  if (!a->q || !a->k_cache || !a->v_cache || !a->page_table || !a->seq_lens || !a->cu_seqlens_q || !a->out) {
    fat_host::set_error("fat_prefill_paged: a required pointer is NULL");
    return FAT_E_INVALID;
  }
  if (a->batch <= 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->total_q < 0 || a->num_pages <= 0 ||
      a->max_pages <= 0) {
    fat_host::set_error("fat_prefill_paged: batch, head counts, num_pages and max_pages must be positive");
    return FAT_E_INVALID;
  }
  if (a->num_heads % a->num_kv_heads != 0) {
    fat_host::set_error("fat_prefill_paged: num_heads %d must be divisible by num_kv_heads %d", a->num_heads,
                        a->num_kv_heads);
    return FAT_E_INVALID;
  }
  if (a->dtype != FAT_DTYPE_F16 && a->dtype != FAT_DTYPE_BF16 && a->dtype != FAT_DTYPE_F32) {
    fat_host::set_error("fat_prefill_paged: dtype must be fp16, bf16 or fp32");
    return FAT_E_UNSUPPORTED;
  }
  const int64_t esz = a->dtype == FAT_DTYPE_F32 ? 4 : 2;  // bytes per element
  if (!valid_prefill_kernel(a->kernel)) {
    fat_host::set_error("fat_prefill_paged: kernel must be FAT_KERNEL_AUTO (0), _PREFILL_PINGPONG (1), "
                        "_PREFILL_4WAVE (2), _PREFILL_4WAVE_SPLIT (3), _PREFILL_WIDE (4) or _PREFILL_GENERIC (5), "
                        "got %d", a->kernel);
    return FAT_E_INVALID;
  }
  const int D = a->head_dim;
  if (D < 16 || D > 512 || (D & (D - 1)) != 0) {
    fat_host::set_error("fat_prefill_paged: head_dim %d unsupported (a power of two from 16 to 512)", D);
    return FAT_E_UNSUPPORTED;
  }
  const int P = a->page_size;
  if (P <= 0 || P > 4096 || (P & (P - 1)) != 0) {
    fat_host::set_error("fat_prefill_paged: page_size %d must be a power of two in [1, 4096]", P);
    return FAT_E_UNSUPPORTED;
  }
  if ((int64_t)a->max_pages * P > 0x7fffffffLL) {
    fat_host::set_error("fat_prefill_paged: max_pages * page_size overflows int32 positions");
    return FAT_E_INVALID;
  }
  if (a->max_seqlen_q < 0) {
    fat_host::set_error("fat_prefill_paged: max_seqlen_q must be non-negative");
    return FAT_E_INVALID;
  }
  if (a->rows != FAT_ROWS_AUTO && a->rows != FAT_ROWS_WIDE && a->rows != FAT_ROWS_LANE) {
    fat_host::set_error("fat_prefill_paged: rows must be FAT_ROWS_AUTO (0), _WIDE (1) or _LANE (2), got %d", a->rows);
    return FAT_E_INVALID;
  }
  const uintptr_t align16 = (uintptr_t)a->q | (uintptr_t)a->k_cache | (uintptr_t)a->v_cache |
                            (uintptr_t)(esz * a->q_stride_t) | (uintptr_t)(esz * a->q_stride_h) |
                            (uintptr_t)(esz * a->k_stride_page) | (uintptr_t)(esz * a->k_stride_slot) |
                            (uintptr_t)(esz * a->k_stride_head) | (uintptr_t)(esz * a->v_stride_page) |
                            (uintptr_t)(esz * a->v_stride_slot) | (uintptr_t)(esz * a->v_stride_head);
  const uintptr_t align8 =
      (uintptr_t)a->out | (uintptr_t)(esz * a->out_stride_t) | (uintptr_t)(esz * a->out_stride_h);
  if ((align16 & 15) || (align8 & 7)) {
    fat_host::set_error("fat_prefill_paged: q and cache rows must be 16-byte aligned and out rows 8-byte aligned");
    return FAT_E_INVALID;
  }
  const int64_t stage_rows = paged_stage_rows(a);
  if (a->kernel == FAT_KERNEL_PREFILL_WIDE && (stage_rows == 0 || !a->workspace)) {
    fat_host::set_error("fat_prefill_paged: the wide prefill kernel runs paged launches on packed copies of K/V "
                        "only (fp16/bf16, head_dim 128, long chunks, and the workspace of "
                        "fat_prefill_paged_workspace_bytes)");
    return FAT_E_UNSUPPORTED;
  }
  if (a->workspace && ((uintptr_t)a->workspace & 255)) {
    fat_host::set_error("fat_prefill_paged: workspace must be 256-byte aligned");
    return FAT_E_INVALID;
  }
  if (a->max_seqlen_q == 0 || a->total_q == 0) return FAT_OK;  // nothing to compute

  fat::PrefillParams prm{};
  prm.q = static_cast<const uint8_t*>(a->q);
  prm.k = static_cast<const uint8_t*>(a->k_cache);
  prm.v = static_cast<const uint8_t*>(a->v_cache);
  prm.cu_q = a->cu_seqlens_q;
  prm.cu_k = nullptr;
  prm.out = static_cast<uint8_t*>(a->out);
  prm.q_st = a->q_stride_t;
  prm.q_sh = a->q_stride_h;
  prm.k_st = a->k_stride_slot;
  prm.k_sh = a->k_stride_head;
  prm.v_st = a->v_stride_slot;
  prm.v_sh = a->v_stride_head;
  prm.o_st = a->out_stride_t;
  prm.o_sh = a->out_stride_h;
  prm.B = a->batch;
  prm.H = a->num_heads;
  prm.Hkv = a->num_kv_heads;
  prm.group = a->num_heads / a->num_kv_heads;
  prm.pt = a->page_table;
  prm.lens = a->seq_lens;
  prm.pt_sb = a->page_table_stride;
  prm.k_sp = a->k_stride_page;
  prm.v_sp = a->v_stride_page;
  prm.pshift = __builtin_ctz((unsigned)P);
  prm.num_pages = a->num_pages;
  prm.max_pages = a->max_pages;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const int64_t kv_bound = (int64_t)a->max_pages * P;  // longest context the table can hold
  if (stage_rows > 0 && a->workspace) {
    // Packed copies of the used K/V rows, then the packed wide kernel on them.
    const PagedStageLayout L = paged_stage_layout(a, stage_rows);
    uint8_t* ws = static_cast<uint8_t*>(a->workspace);
    int32_t* cu_k = reinterpret_cast<int32_t*>(ws);
    const int rc = fat_host::launch_paged_stage(prm, D, a->batch, (int)kv_bound, cu_k, ws + L.k, ws + L.v, stream);
    if (rc != FAT_OK) return rc;
    fat::PrefillParams pk = prm;
    pk.k = ws + L.k;
    pk.v = ws + L.v;
    pk.cu_k = cu_k;
    pk.k_st = pk.v_st = (int64_t)a->num_kv_heads * D;
    pk.k_sh = pk.v_sh = D;
    pk.pt = nullptr;
    pk.lens = nullptr;
    return launch_prefill<0>(pk, a->max_seqlen_q, kv_bound, a->dtype, D, a->causal != 0, a->softmax_scale,
                             FAT_KERNEL_PREFILL_WIDE, "fat_prefill_paged", stream,
                             L.total > L.vpre ? ws + L.vpre : nullptr, (int)stage_rows, a->total_q);
  }
  // One load covers 256 / (D / 8) rows (16 at D128, 32 at D64): with pages at
  // least that long its rows share a page and the page id is wave-uniform.
  bool uniform = P >= 256 / (D / 8);
  // Byte offset past the last row of the pool, from a KV head's first row:
  // below 2^31 the uniform loads address the pool as one buffer (PG 3).
  const int64_t kspan =
      (int64_t)(a->num_pages - 1) * 2 * a->k_stride_page + (int64_t)(P - 1) * 2 * a->k_stride_slot + 2 * D;
  const int64_t vspan =
      (int64_t)(a->num_pages - 1) * 2 * a->v_stride_page + (int64_t)(P - 1) * 2 * a->v_stride_slot + 2 * D;
  bool off32 = kspan < 0x7fffffffLL && vspan < 0x7fffffffLL;
  // `rows` forces the per-lane variant (FAT_ROWS_LANE) or the uniform one
  // with 64-bit row addresses (FAT_ROWS_WIDE); all three give identical bits.
  if (a->rows == FAT_ROWS_LANE) uniform = false;
  else if (a->rows == FAT_ROWS_WIDE) off32 = false;
  if (uniform && off32)
    return launch_prefill<3>(prm, a->max_seqlen_q, kv_bound, a->dtype, D, a->causal != 0, a->softmax_scale,
                             a->kernel, "fat_prefill_paged", stream);
  if (uniform)
    return launch_prefill<2>(prm, a->max_seqlen_q, kv_bound, a->dtype, D, a->causal != 0, a->softmax_scale,
                             a->kernel, "fat_prefill_paged", stream);
  return launch_prefill<1>(prm, a->max_seqlen_q, kv_bound, a->dtype, D, a->causal != 0, a->softmax_scale,
                           a->kernel, "fat_prefill_paged", stream);
}
