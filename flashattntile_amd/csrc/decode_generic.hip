// decode_generic.hip -- paged decode for the shapes the VALU and MFMA decode
// kernels (decode.hip) do not take: fp32 queries and caches, page sizes that
// are not a power of two or are below the rows one 16-byte load per lane
// covers, and head_dim 16, 32, 256 or 512.
//
// Semantics are those of the other decode kernels and of the reference's
// native decode (csrc/paged_decode.cu:80-235): one query per sequence, query
// head h reads KV head h / group, a sequence of length <= 0 yields zeros,
// int8/fp8 pages are dequantised as the other decode kernels do (K with fp16
// queries exact in fp32 with k_scale, everything else rounded to the query
// type, flashattn_tile/quant.py:145-161), and scores, softmax and PV run in
// fp32.
//
// Design: one workgroup of 256 threads per (partition, KV head, up to 8 of
// its query heads, sequence) streams 32-token tiles.
//   * every thread loads 16-byte chunks of the tile's K and V rows (row-
//     coalesced; the page id is looked up per row, so any page size works)
//     one tile ahead into registers, then writes them to LDS as fp32;
//   * thread (head, row) takes the whole q.k dot product of one (query head,
//     token) pair from LDS; a 32-lane shuffle gives each head's tile max and
//     sum for the online softmax;
//   * thread (head, dims) accumulates its output dims over the tile's 32 rows
//     (at head_dim 16 the 8 heads x 16 dims leave half the threads idle).
// Three barriers per tile.  It is an HBM-streaming kernel like the others,
// but it spends more VALU and LDS work per byte; the fast kernels keep every
// shape they support.
#include "decode_params.h"

namespace fat {

template <typename QT, int KV, int D>
__global__ __launch_bounds__(256) void paged_decode_generic_kernel(const DecodeParams p, int heads_per_wg) {
  constexpr int NT = 256;
  constexpr int TR = 32;                                   // tokens per tile
  constexpr int HM = fat_host::kGenericHeads;              // query heads per workgroup (max)
  constexpr int EB = KV == KV_SAME ? Elem<QT>::kBytes : 1; // bytes per stored element
  constexpr int EPC = 16 / EB;                             // elements per 16-byte chunk
  constexpr int CPR = D / EPC;                             // chunks per row
  constexpr int NCH = TR * CPR;                            // chunks per tile of K (or V)
  constexpr int CPT = (NCH + NT - 1) / NT;                 // chunks per thread
  constexpr int KRS = D + 1;                               // LDS K row stride (floats)
  constexpr int OPT = (HM * D + NT - 1) / NT;              // output values per thread
  static_assert(CPR >= 1 && CPR * EPC == D, "unsupported head_dim / element size");
  static_assert(OPT * NT == HM * D || (OPT == 1 && HM * D < NT), "unsupported head_dim");

  __shared__ float sK[TR * KRS];
  __shared__ float sV[TR * D];
  __shared__ float sQ[HM * D];
  __shared__ float sP[HM][TR];
  __shared__ float sAlpha[HM];
  __shared__ float sML[HM][2];

  const int tid = threadIdx.x;
  const int split = blockIdx.x;
  const int S = gridDim.x;
  const int y = blockIdx.y;
  const int b = blockIdx.z;
  const int hpw = heads_per_wg;
  const int subs = (p.group + hpw - 1) / hpw;
  const int sub = y % subs;
  const int kvh = y / subs;
  const int head0 = kvh * p.group + sub * hpw;
  const int nvalid = min(hpw, p.group - sub * hpw);

  // Partition of this sequence's pages (kernels/decode.py:271-276 semantics).
  const int64_t cap = (int64_t)p.max_pages * p.P;
  const int seq_len = (int)max((int64_t)0, min((int64_t)p.lens[b], cap));
  const int np = (seq_len + p.P - 1) / p.P;
  const int pps = p.pps_fixed > 0 ? p.pps_fixed : (np + S - 1) / S;
  const int pb = min(np, split * pps);
  const int pe = split == S - 1 ? np : min(np, pb + pps);
  const int t_begin = pb * p.P;
  const int t_end = min(seq_len, pe * p.P);
  const int n_tiles = t_end > t_begin ? (t_end - t_begin + TR - 1) / TR : 0;

  // q of the workgroup's heads as fp32 (padded head slots repeat head0).
  for (int i = tid; i < HM * D; i += NT) {
    const int hs = i / D;
    const int d = i - hs * D;
    const int h = head0 + (hs < nvalid ? hs : 0);
    const int64_t qi = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + d;
    if constexpr (std::is_same<QT, F32>::value) {
      sQ[i] = reinterpret_cast<const float*>(p.q)[qi];
    } else {
      sQ[i] = Pair<QT>::lo((u32)reinterpret_cast<const uint16_t*>(p.q)[qi]);
    }
  }

  const int32_t* ptrow = p.pt + (int64_t)b * p.pt_sb;
  u32x4 kr[CPT], vr[CPT];
  float ksc[CPT], vsc[CPT];
  // Chunks of tile `tile` into registers.  Rows past t_end re-read the last
  // valid token (finite data); their scores are masked.
  auto fetch = [&](int tile) {
    const int t0 = t_begin + tile * TR;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int ci = tid + j * NT;
      if (NCH % NT != 0 && ci >= NCH) break;
      const int row = ci / CPR;
      const int cc = ci - row * CPR;
      const int tok = min(t0 + row, t_end - 1);
      const int lp = tok / p.P;
      const int slot = tok - lp * p.P;
      const int phys = min(max(ptrow[lp], 0), p.num_pages - 1);
      const int64_t ko = (int64_t)phys * p.k_sp + (int64_t)slot * p.k_ss + (int64_t)kvh * p.k_sh + cc * EPC;
      const int64_t vo = (int64_t)phys * p.v_sp + (int64_t)slot * p.v_ss + (int64_t)kvh * p.v_sh + cc * EPC;
      kr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.k + EB * ko));  // read once
      vr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.v + EB * vo));
      if constexpr (KV != KV_SAME) {
        ksc[j] = p.ks[(int64_t)phys * p.sc_sp + (int64_t)kvh * p.sc_sh];
        vsc[j] = p.vs[(int64_t)phys * p.sc_sp + (int64_t)kvh * p.sc_sh];
      }
    }
  };
  // One chunk as EPC fp32 values.  8-bit codes dequantise as the VALU and
  // MFMA decode kernels do: K with fp16 queries stays float(x) * k_scale in
  // fp32 (the reference's quantised kernel, kernels/decode.py:419-429), every
  // other dequantised value is round_to_QT(float(x) * scale) (its
  // dequantise-then-attend path, kernels/decode.py:674-682; quant.py:145-161).
  auto unpack = [&](const u32x4& raw, float sc, float* f, bool round_to_q) {
    if constexpr (KV == KV_SAME && std::is_same<QT, F32>::value) {
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = as_f32(raw[e]);
    } else if constexpr (KV == KV_SAME) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = Pair<QT>::lo(raw[e]);
        f[2 * e + 1] = Pair<QT>::hi(raw[e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x[4];
        if constexpr (KV == KV_I8) {
          i8x4_biased(raw[e], x);  // x + 128, exact
#pragma unroll
          for (int u = 0; u < 4; ++u) x[u] = (x[u] - 128.0f) * sc;
        } else {
          fp8x4(raw[e], x);
#pragma unroll
          for (int u = 0; u < 4; ++u) x[u] = x[u] * sc;
        }
        if (round_to_q) {
          const u32 w0 = Pair<QT>::pack(x[0], x[1]);
          const u32 w1 = Pair<QT>::pack(x[2], x[3]);
          x[0] = Pair<QT>::lo(w0);
          x[1] = Pair<QT>::hi(w0);
          x[2] = Pair<QT>::lo(w1);
          x[3] = Pair<QT>::hi(w1);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) f[4 * e + u] = x[u];
      }
    }
  };

  // Score role: (head slot hs, tile row).  Output role: OPT (head, dim) pairs.
  const int srow = tid & (TR - 1);
  const int shs = tid / TR;
  float m_run = -INFINITY, l_run = 0.f;  // of head slot shs (log2 units)
  float acc[OPT];
#pragma unroll
  for (int k = 0; k < OPT; ++k) acc[k] = 0.f;

  if (n_tiles > 0) fetch(0);
  for (int tile = 0; tile < n_tiles; ++tile) {
    __syncthreads();  // the previous tile's readers are done with sK / sV / sP
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int ci = tid + j * NT;
      if (NCH % NT != 0 && ci >= NCH) break;
      const int row = ci / CPR;
      const int cc = ci - row * CPR;
      float f[EPC];
      unpack(kr[j], KV != KV_SAME ? ksc[j] : 1.f, f, !std::is_same<QT, F16>::value);
#pragma unroll
      for (int e = 0; e < EPC; ++e) sK[row * KRS + cc * EPC + e] = f[e];
      unpack(vr[j], KV != KV_SAME ? vsc[j] : 1.f, f, true);
#pragma unroll
      for (int e = 0; e < EPC; ++e) sV[row * D + cc * EPC + e] = f[e];
    }
    if (tile + 1 < n_tiles) fetch(tile + 1);
    __syncthreads();

    // ---- scores and the online softmax of head slot shs ----
    if (shs < nvalid) {
      const float* kq = &sK[srow * KRS];
      const float* qq = &sQ[shs * D];
      float s = 0.f;
#pragma unroll 8
      for (int d = 0; d < D; ++d) s = __builtin_fmaf(qq[d], kq[d], s);
      const bool valid = t_begin + tile * TR + srow < t_end;
      s = valid ? s * p.scale_log2 : -INFINITY;
      float mx = s;
#pragma unroll
      for (int off = TR / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      const float m_new = fmaxf(m_run, mx);
      // m_new is finite: every tile holds at least one valid row.
      const float alpha = fast_exp2(m_run - m_new);
      const float pr = valid ? fast_exp2(s - m_new) : 0.f;
      float ps = pr;
#pragma unroll
      for (int off = TR / 2; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
      l_run = l_run * alpha + ps;
      m_run = m_new;
      sP[shs][srow] = pr;
      if (srow == 0) sAlpha[shs] = alpha;
    }
    __syncthreads();

    // ---- acc = acc * alpha + P V over the tile ----
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int idx = tid + k * NT;
      const int hs = idx / D;
      const int d = idx - hs * D;
      if (hs < nvalid) {
        float a = acc[k] * sAlpha[hs];
#pragma unroll 8
        for (int r = 0; r < TR; ++r) a = __builtin_fmaf(sP[hs][r], sV[r * D + d], a);
        acc[k] = a;
      }
    }
  }

  if (srow == 0 && shs < HM) {
    sML[shs][0] = m_run;
    sML[shs][1] = l_run;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int idx = tid + k * NT;
    const int hs = idx / D;
    const int d = idx - hs * D;
    if (hs >= nvalid) continue;
    const int h = head0 + hs;
    const float L = n_tiles > 0 ? sML[hs][1] : 0.f;
    if (S == 1) {
      store_elem<QT>(p.out, (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + d, L > 0.f ? acc[k] / L : 0.f);
    } else {
      const int64_t row = ((int64_t)b * p.H + h) * S + split;
      p.ws_acc[row * D + d] = acc[k];
      if (d == 0) {
        p.ws_ml[row * 2 + 0] = n_tiles > 0 ? sML[hs][0] : -INFINITY;
        p.ws_ml[row * 2 + 1] = L;
      }
    }
  }
}

}  // namespace fat

namespace {

template <typename QT, int KV>
int launch_generic_kv(const fat::DecodeParams& prm, int D, int hpw, dim3 grid, hipStream_t stream) {
  switch (D) {
    case 16:
      hipLaunchKernelGGL((fat::paged_decode_generic_kernel<QT, KV, 16>), grid, dim3(256), 0, stream, prm, hpw);
      break;
    case 32:
      hipLaunchKernelGGL((fat::paged_decode_generic_kernel<QT, KV, 32>), grid, dim3(256), 0, stream, prm, hpw);
      break;
    case 64:
      hipLaunchKernelGGL((fat::paged_decode_generic_kernel<QT, KV, 64>), grid, dim3(256), 0, stream, prm, hpw);
      break;
    case 128:
      hipLaunchKernelGGL((fat::paged_decode_generic_kernel<QT, KV, 128>), grid, dim3(256), 0, stream, prm, hpw);
      break;
    case 256:
      hipLaunchKernelGGL((fat::paged_decode_generic_kernel<QT, KV, 256>), grid, dim3(256), 0, stream, prm, hpw);
      break;
    case 512:
      hipLaunchKernelGGL((fat::paged_decode_generic_kernel<QT, KV, 512>), grid, dim3(256), 0, stream, prm, hpw);
      break;
    default:
      fat_host::set_error("fat_paged_decode: head_dim %d unsupported (a power of two from 16 to 512)", D);
      return FAT_E_UNSUPPORTED;
  }
  return fat_host::launch_status("paged_decode_generic_kernel");
}

template <typename QT>
int launch_generic_q(const fat::DecodeParams& prm, int kv, int D, int hpw, dim3 grid, hipStream_t stream) {
  switch (kv) {
    case fat::KV_SAME: return launch_generic_kv<QT, fat::KV_SAME>(prm, D, hpw, grid, stream);
    case fat::KV_I8: return launch_generic_kv<QT, fat::KV_I8>(prm, D, hpw, grid, stream);
    default: return launch_generic_kv<QT, fat::KV_FP8>(prm, D, hpw, grid, stream);
  }
}

}  // namespace

namespace fat_host {

int launch_decode_generic(const fat::DecodeParams& prm, int q_dtype, int kv, int head_dim, int heads_per_wg,
                          dim3 grid, hipStream_t stream) {
  if (heads_per_wg < 1 || heads_per_wg > kGenericHeads) {
    set_error("fat_paged_decode: generic decode takes 1..%d heads per workgroup, got %d", kGenericHeads,
              heads_per_wg);
    return FAT_E_INVALID;
  }
  if (q_dtype == FAT_DTYPE_F32) {
    if (kv != fat::KV_SAME) {
      set_error("fat_paged_decode: fp32 queries take an fp32 cache");
      return FAT_E_UNSUPPORTED;
    }
    return launch_generic_kv<fat::F32, fat::KV_SAME>(prm, head_dim, heads_per_wg, grid, stream);
  }
  if (q_dtype == FAT_DTYPE_F16) return launch_generic_q<fat::F16>(prm, kv, head_dim, heads_per_wg, grid, stream);
  return launch_generic_q<fat::BF16>(prm, kv, head_dim, heads_per_wg, grid, stream);
}

}  // namespace fat_host
