/*
 * fat_abi.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * The shared library libfat_hip.so exports exactly the functions declared
 * here.  Every entry point takes plain device pointers, element strides and
 * sizes; no framework types cross this boundary.  The caller owns every
 * buffer (inputs, outputs and the split-K workspace); the library never
 * allocates, frees or synchronises, and enqueues its kernels on the
 * hipStream_t passed as `stream` (NULL = the default stream).
 *
 * Return value: 0 on success, otherwise a FAT_E_* code; the matching message
 * is available from fat_last_error() on the calling thread.
 *
 * Reference interfaces replaced (paths relative to the FlashAttnTile tree):
 *   fat_paged_decode       flashattn_tile/kernels/decode.py:533-642
 *                          (paged_decode_attention: _decode_paged_kernel,
 *                          _decode_paged_split_kernel + _decode_reduce_kernel)
 *                          and csrc/paged_decode.cu:297-344 (paged_decode_cuda,
 *                          bound by csrc/bindings.cpp:14-20)
 *   fat_paged_decode (int8/fp8 kv_dtype)
 *                          flashattn_tile/kernels/decode.py:645-704
 *                          (paged_decode_attention_fp8: _decode_paged_quant_kernel)
 *   fat_prefill_varlen     flashattn_tile/kernels/prefill.py:236-326
 *                          (prefill_attention: _fwd_varlen_kernel)
 *   fat_prefill_paged      no reference counterpart: the paged (chunked)
 *                          prefill that flashattn_tile/backend.py:158-162
 *                          lacks (it requires packed K/V); semantics of
 *                          flashattn_tile/kernels/prefill.py:35-138 with K/V
 *                          read through the page table
 *   fat_quantize_pages     flashattn_tile/quant.py:84-142
 *                          (quantize_kv_pages, one of K or V per call)
 *   fat_append_kv          flashattn_tile/paging.py:172-210
 *                          (append_tokens), plus the requantisation of the
 *                          touched pages of an int8/fp8 copy of the cache
 *   fat_cache_stats        the device reductions of validate_cache,
 *                          flashattn_tile/paging.py:84-130 (as called by
 *                          flashattn_tile/kernels/decode.py:503-522)
 */
#ifndef FAT_ABI_H
#define FAT_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 14: fat_decode_args.merge_counters and fat_paged_decode_counters_bytes:
 *     split-K decode merges its partitions inside the decode launch.
 * 13: fat_cache_stats (paged-cache validation in one launch).
 * 12: fat_prefill_paged_args.workspace and
 *     fat_prefill_paged_workspace_bytes: long paged prefill chunks run on
 *     the wide kernel through packed copies of their K/V rows.
 * 11: fat_prefill_varlen_workspace_bytes (the workspace one launch uses);
 *     the bf16 V pre-pass scales V per (sequence, KV head);
 *     FAT_KERNEL_PREFILL_WIDE; fp32 prefill and head_dim 16..512
 *     (FAT_KERNEL_PREFILL_GENERIC); decode head_dim 16 and 512 (generic
 *     decode kernel).
 * 10: fat_prefill_workspace_bytes is non-zero: bf16 fat_prefill_varlen
 *     uses the workspace for an fp16 copy of V (optional).
 * 9: fat_paged_decode_noalloc (allocation-free decode).
 * 8: fp32 decode, any page size and head_dim 32/256 through the generic
 *    decode kernel (FAT_KERNEL_DECODE_GENERIC); the paged prefill `rows`
 *    field replaces the library's environment overrides. */
#define FAT_ABI_VERSION 14

/* Element types understood by the kernels. */
enum fat_dtype {
  FAT_DTYPE_F16 = 0,     /* IEEE binary16                                  */
  FAT_DTYPE_BF16 = 1,    /* bfloat16                                       */
  FAT_DTYPE_I8 = 2,      /* symmetric int8 KV storage (scale = absmax/127) */
  FAT_DTYPE_FP8E4M3 = 3, /* OCP float8 e4m3fn KV storage (absmax/448)      */
  FAT_DTYPE_F32 = 4      /* IEEE binary32 (decode q/K/V/out, and the
                            fat_quantize_pages source)                     */
};

/* Kernel choice (the `kernel` field of the decode and prefill arguments).
 * FAT_KERNEL_AUTO lets the library choose from the shape; the others force
 * one kernel family, e.g. the winner a tuning run stored for this shape. */
enum fat_kernel {
  FAT_KERNEL_AUTO = 0,
  FAT_KERNEL_DECODE_VALU = 1,      /* one query per sequence (q_len <= 1)     */
  FAT_KERNEL_DECODE_MFMA = 2,      /* any cache dtype and q_len               */
  FAT_KERNEL_DECODE_GENERIC = 3,   /* one query per sequence; every dtype,
                                      page size and head_dim the ABI takes   */
  FAT_KERNEL_PREFILL_PINGPONG = 1, /* 8 waves, 256 query rows per workgroup   */
  FAT_KERNEL_PREFILL_4WAVE = 2,    /* 4 waves, 128 query rows per workgroup   */
  FAT_KERNEL_PREFILL_4WAVE_SPLIT = 3, /* 8 waves, 128 query rows: two 4-wave
                                         groups take alternate key tiles and
                                         merge (m, l, O) at the end         */
  FAT_KERNEL_PREFILL_WIDE = 4, /* 8 waves x 64 query rows (512 per workgroup):
                                  packed fat_prefill_varlen at head_dim 128;
                                  bf16 needs the workspace (an fp16 copy of
                                  V), other shapes return FAT_E_UNSUPPORTED */
  FAT_KERNEL_PREFILL_GENERIC = 5 /* fp32 VALU kernel for every dtype and
                                    power-of-two head_dim 16..512; the only
                                    kernel for fp32 and head_dim 16 / 512 */
};

/* Row addressing of fat_prefill_paged (the `rows` field): AUTO picks the
 * fastest form the page size allows; the others force one (tests check that
 * all of them give identical bits). */
enum fat_rows {
  FAT_ROWS_AUTO = 0,
  FAT_ROWS_WIDE = 1, /* wave-uniform page ids, 64-bit row addresses          */
  FAT_ROWS_LANE = 2  /* per-lane page ids and row addresses (any page size)  */
};

/* Error codes. */
enum fat_status {
  FAT_OK = 0,
  FAT_E_INVALID = 1,     /* bad argument (shape, dtype, pointer, stride)   */
  FAT_E_UNSUPPORTED = 2, /* valid request this build has no kernel for     */
  FAT_E_LAUNCH = 3       /* the HIP runtime rejected a launch              */
};

/*
 * Paged decode: one query per sequence against a paged K/V cache.
 *
 * Layouts (NHD pages, flashattn_tile/paging.py:1-20):
 *   q        [batch, num_heads, head_dim]          q_dtype (fp16, bf16, fp32)
 *   k_cache  [num_pages, page_size, num_kv_heads, head_dim]  kv_dtype
 *   v_cache  same shape and dtype as k_cache
 *   k_scale  [num_pages, num_kv_heads] fp32, only for int8/fp8 kv_dtype
 *   v_scale  same as k_scale
 *   page_table int32 [batch, max_pages]  (row stride page_table_stride)
 *   seq_lens int32 [batch]; a sequence of length <= 0 yields zeros, and
 *            lengths beyond max_pages*page_size are clamped to it
 * head_dim is a power of two from 16 to 512 and page_size any positive number (page
 * ids are clamped to [0, num_pages)).  The VALU and MFMA kernels take
 * fp16/bf16 queries, head_dim 64 or 128 and power-of-two pages of at least
 * the rows one 16-byte load per lane covers: 4 (fp16/bf16, head_dim 128), 8
 * (fp16/bf16 64; int8/fp8 128) or 16 (int8/fp8 64).  Every other request
 * runs on the generic kernel (one query per sequence only); fp32 queries
 * take an fp32 cache.
 *   out      [batch, num_heads, head_dim]          q_dtype
 * Strides are in elements; the head_dim axis must be contiguous.
 *
 * Query head h reads KV head h / (num_heads / num_kv_heads).  The context of
 * sequence b is split into split_k partitions.  With pages_per_split == 0 each
 * holds ceil(ceil(len/P)/split_k) pages (the reference's split kernel,
 * flashattn_tile/kernels/decode.py:271-276); with pages_per_split > 0 every
 * partition holds that many pages, so work per workgroup is the same for
 * short and long sequences of a ragged batch (partitions past a sequence's
 * end are empty, and the last partition takes any pages beyond
 * split_k * pages_per_split).  With split_k > 1 the partitions are merged by
 * a log-sum-exp reduction through `workspace`, which must hold
 * fat_paged_decode_workspace_bytes(batch, num_heads, head_dim, split_k) bytes
 * (it may be NULL when split_k == 1).  int8/fp8 pages: with bf16 queries
 * K and V are dequantised as round_to_bf16(float(x) * scale), as
 * dequantize_kv_pages (flashattn_tile/quant.py:145-161) followed by the fp32
 * reference does.  With fp16 queries k_scale multiplies the fp32 scores of
 * the exact 8-bit K, as the reference's quantised kernel does
 * (flashattn_tile/kernels/decode.py:419-429), fp8 V is round_to_fp16(
 * float(x) * scale) and int8 V is x * fp16(scale), within one fp16 ulp of
 * it; the results stay within the dequantise-then-attend tolerance.
 */
typedef struct fat_decode_args {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const float* k_scale;
  const float* v_scale;
  const int32_t* page_table;
  const int32_t* seq_lens;
  void* out;
  void* workspace;
  int64_t q_stride_b, q_stride_h;
  int64_t k_stride_page, k_stride_slot, k_stride_head;
  int64_t v_stride_page, v_stride_slot, v_stride_head;
  int64_t scale_stride_page, scale_stride_head;
  int64_t page_table_stride;
  int64_t out_stride_b, out_stride_h;
  int32_t batch;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t num_pages;
  int32_t max_pages;
  int32_t split_k;
  int32_t waves_per_group; /* 0 = chosen by the library, else 4 or 8 */
  int32_t q_dtype;  /* FAT_DTYPE_F16, _BF16 or _F32 (also the out dtype)  */
  int32_t kv_dtype; /* q_dtype, or FAT_DTYPE_I8 / _FP8E4M3 (16-bit q)    */
  int32_t pages_per_split; /* 0 = ceil(pages / split_k) per sequence        */
  float softmax_scale;
  /* Multi-token decode (q_len > 1): q and out are [batch, q_len, num_heads,
   * head_dim] with token strides q_stride_t / out_stride_t; token t of
   * sequence b sees keys j <= seq_lens[b] - q_len + t (bottom-right causal,
   * as fat_prefill_paged).  q_len 0 or 1 is single-query decode and the
   * token strides are ignored.  The split-K workspace then holds
   * batch * q_len rows: size it with fat_paged_decode_workspace_bytes(
   * batch * q_len, ...).  At most 64 tokens. */
  int64_t q_stride_t, out_stride_t;
  int32_t q_len;
  int32_t kernel; /* FAT_KERNEL_AUTO, _DECODE_VALU, _MFMA or _GENERIC */
  /* Optional (split_k > 1): int32 counters, one per (sequence, query head),
   * fat_paged_decode_counters_bytes(batch * q_len, num_heads) bytes, all
   * zero before the first launch that uses them; every launch leaves them
   * zero.  With them the VALU and MFMA kernels merge the partitions in the
   * decode launch itself (the last partition of each head group to finish
   * merges them, with the arithmetic of the merge kernel: bit-identical
   * results) when split_k <= 16 and a workgroup's heads make at most two
   * output elements per thread (the last workgroup merges alone); otherwise
   * (NULL, more partitions or heads, the generic kernel) a second kernel
   * merges and the counters are not touched.  Launches that may run at the
   * same time (other streams) must not share counters. */
  int32_t* merge_counters;
} fat_decode_args;

/*
 * Packed varlen prefill (flash attention forward).
 *   q   [total_q, num_heads, head_dim]      dtype
 *   k,v [total_k, num_kv_heads, head_dim]   dtype
 *   cu_seqlens_q / cu_seqlens_k int32 [batch + 1], starting at 0,
 *   non-decreasing, kv_len >= q_len per sequence when causal.
 *   out [total_q, num_heads, head_dim]      dtype
 * dtype is fp16, bf16 or fp32; head_dim a power of two from 16 to 512.
 * fp32 and head_dim 16 / 512 run on the generic kernel only
 * (FAT_KERNEL_AUTO or FAT_KERNEL_PREFILL_GENERIC); head_dim 256 at fp16 /
 * bf16 on the 4-wave kernel (or the generic one); a kernel that does not
 * take the shape returns FAT_E_UNSUPPORTED.  The same holds for
 * fat_prefill_paged.
 * Causal masking is bottom-right aligned: query i of a sequence sees key j
 * iff j <= i + (kv_len - q_len)  (flashattn_tile/reference.py:19-22).
 * `workspace` is optional: NULL, or 256-byte aligned and holding
 * fat_prefill_varlen_workspace_bytes(args) bytes (at most
 * fat_prefill_workspace_bytes(total_k, num_kv_heads, head_dim)).  Only bf16
 * launches on the large-grid kernel whose sequences average at least 2048
 * query tokens use it (the query returns 0 otherwise): a pre-pass writes an
 * fp16 copy of V there, scaled by one power of two per (sequence, KV head),
 * and the kernel stages that copy (results within the same bound as the
 * in-kernel conversion it replaces).  Without the workspace the kernel
 * converts V tile by tile.
 */
typedef struct fat_prefill_args {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* cu_seqlens_q;
  const int32_t* cu_seqlens_k;
  void* out;
  void* workspace;
  int64_t q_stride_t, q_stride_h;
  int64_t k_stride_t, k_stride_h;
  int64_t v_stride_t, v_stride_h;
  int64_t out_stride_t, out_stride_h;
  int32_t batch;
  int32_t total_q;
  int32_t total_k;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t max_seqlen_q;
  int32_t max_seqlen_k;
  int32_t causal;
  int32_t dtype; /* FAT_DTYPE_F16, FAT_DTYPE_BF16 or FAT_DTYPE_F32 */
  float softmax_scale;
  int32_t kernel; /* FAT_KERNEL_AUTO or a FAT_KERNEL_PREFILL_* */
} fat_prefill_args;

/*
 * Paged (chunked) prefill: the packed queries of each sequence attend to the
 * sequence's keys in a paged K/V cache.
 *   q   [total_q, num_heads, head_dim]                     dtype
 *   k_cache, v_cache [num_pages, page_size, num_kv_heads, head_dim]  dtype
 *   page_table int32 [batch, max_pages], seq_lens int32 [batch]: key j of
 *   sequence b is slot j % page_size of page page_table[b, j / page_size],
 *   for j < kv_len = seq_lens[b] (the chunk's own keys included).
 *   cu_seqlens_q int32 [batch + 1], starting at 0, non-decreasing;
 *   kv_len >= q_len per sequence when causal.
 *   out [total_q, num_heads, head_dim]                     dtype
 * Causal masking is bottom-right aligned, as fat_prefill_varlen: query i of
 * a sequence sees key j iff j <= i + (kv_len - q_len).  page_size must be a
 * power of two.  Page ids are clamped to [0, num_pages) and kv_len to
 * max_pages * page_size on the device, so a bad table gives a wrong answer,
 * never an out-of-bounds read.
 * `workspace` is optional: NULL, or 256-byte aligned and holding
 * fat_prefill_paged_workspace_bytes(args) bytes.  When that is non-zero
 * (fp16/bf16, head_dim 128, chunks averaging thousands of queries) the
 * launch first copies the used K/V rows out of the pages into the workspace
 * and runs the packed wide kernel on the copies (`rows` then has no
 * effect); without the workspace it runs the paged kernels.  Same results
 * up to the kernels' rounding (each within the prefill tolerance).
 */
typedef struct fat_prefill_paged_args {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* page_table;
  const int32_t* seq_lens;
  const int32_t* cu_seqlens_q;
  void* out;
  int64_t q_stride_t, q_stride_h;
  int64_t k_stride_page, k_stride_slot, k_stride_head;
  int64_t v_stride_page, v_stride_slot, v_stride_head;
  int64_t page_table_stride;
  int64_t out_stride_t, out_stride_h;
  int32_t batch;
  int32_t total_q;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t num_pages;
  int32_t max_pages;
  int32_t max_seqlen_q;
  int32_t causal;
  int32_t dtype; /* FAT_DTYPE_F16, FAT_DTYPE_BF16 or FAT_DTYPE_F32 */
  float softmax_scale;
  int32_t kernel; /* FAT_KERNEL_AUTO or a FAT_KERNEL_PREFILL_* (WIDE: with
                     the staging workspace only)                           */
  int32_t rows;   /* FAT_ROWS_AUTO, _WIDE or _LANE                        */
  void* workspace; /* optional, see above                                 */
} fat_prefill_paged_args;

/*
 * Per-(page, KV head) quantisation of a paged cache tensor.
 *   src   [num_pages, page_size, num_kv_heads, head_dim]  src_dtype
 *   dst   same shape                                       dst_dtype
 *   scale fp32 [num_pages, num_kv_heads]
 * For every (page, head): scale = max(absmax over (slot, dim) / qmax, 1e-8)
 * with qmax = 127 (int8) or 448 (fp8); the division is correctly rounded.
 * int8 codes are clamp(round_half_even(x / scale), -127, 127); fp8 codes are
 * clamp(x / scale, -448, 448) rounded to nearest-even e4m3fn
 * (flashattn_tile/quant.py:114-127).  Strides are in elements and head_dim is
 * contiguous.  Source values must be finite.
 */
typedef struct fat_quantize_args {
  const void* src;
  void* dst;
  float* scale;
  int64_t src_stride_page, src_stride_slot, src_stride_head;
  int64_t dst_stride_page, dst_stride_slot, dst_stride_head;
  int64_t scale_stride_page, scale_stride_head;
  int32_t num_pages;
  int32_t page_size;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t src_dtype; /* FAT_DTYPE_F16, FAT_DTYPE_BF16 or FAT_DTYPE_F32 */
  int32_t dst_dtype; /* FAT_DTYPE_I8 or FAT_DTYPE_FP8E4M3 */
} fat_quantize_args;

/*
 * Append one token per sequence to a paged cache (and its quantised copy).
 *   new_k, new_v   [batch, num_kv_heads, head_dim]       dtype
 *   k_cache, v_cache [num_pages, page_size, num_kv_heads, head_dim]  dtype
 *   page_table     int32 [batch, max_pages], seq_lens int32 [batch]
 * Token b goes to slot seq_lens[b] % page_size of page
 * page_table[b, seq_lens[b] / page_size].  With advance != 0, seq_lens[b]
 * is incremented after every write of the call is done.
 * Optional quantised copy (quant_k_cache/quant_v_cache non-NULL, int8 or fp8
 * pages with fp32 scales [num_pages, num_kv_heads]): every (page, KV head)
 * that received a token is requantised from the updated dtype page, so the
 * copy holds what fat_quantize_pages of the whole updated cache would give.
 * The caller guarantees 0 <= seq_lens[b] < max_pages * page_size and page
 * ids in [0, num_pages) (flashattn_tile/paging.py:192-205 checks this on the
 * host); an entry that breaks it is skipped, never written out of bounds.
 * Several sequences may append into the same page (distinct slots).
 */
typedef struct fat_append_args {
  const void* new_k;
  const void* new_v;
  void* k_cache;
  void* v_cache;
  void* quant_k_cache;
  void* quant_v_cache;
  float* k_scale;
  float* v_scale;
  const int32_t* page_table;
  int32_t* seq_lens;
  int64_t new_k_stride_b, new_k_stride_h;
  int64_t new_v_stride_b, new_v_stride_h;
  int64_t k_stride_page, k_stride_slot, k_stride_head;
  int64_t v_stride_page, v_stride_slot, v_stride_head;
  int64_t qk_stride_page, qk_stride_slot, qk_stride_head;
  int64_t qv_stride_page, qv_stride_slot, qv_stride_head;
  int64_t scale_stride_page, scale_stride_head; /* shared by k/v_scale */
  int64_t page_table_stride;
  int32_t batch;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t num_pages;
  int32_t max_pages;
  int32_t dtype;       /* FAT_DTYPE_F16 or FAT_DTYPE_BF16 */
  int32_t quant_dtype; /* FAT_DTYPE_I8 or FAT_DTYPE_FP8E4M3 (with a copy) */
  int32_t advance;     /* 1 = seq_lens += 1 (the reference's behaviour)   */
} fat_append_args;

/* ABI version of the loaded library (FAT_ABI_VERSION at build time). */
int fat_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* fat_last_error(void);

/* Bytes of split-K workspace fat_paged_decode needs (0 when split_k == 1). */
size_t fat_paged_decode_workspace_bytes(int32_t batch, int32_t num_heads,
                                        int32_t head_dim, int32_t split_k);

/* Bytes of fat_decode_args.merge_counters for `rows` = batch * q_len query
 * rows (q_len 1 for single-query decode) of num_heads heads. */
size_t fat_paged_decode_counters_bytes(int32_t rows, int32_t num_heads);

/* Enqueue paged decode (fp16/bf16/fp32/int8/fp8 K/V) on `stream`.
 * Replaces flashattn_tile/kernels/decode.py:533-704 (see file header). */
int fat_paged_decode(const fat_decode_args* args, void* stream);

/* Allocation-free paged decode.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops and harnesses that forbid hipMalloc).  The same launch as
 * fat_paged_decode(args, stream), except that the split-K workspace is a
 * device array inside the library (FAT_DECODE_NOALLOC_MAX_WORKSPACE bytes
 * per GPU, held until the process ends); args->workspace and
 * args->merge_counters are ignored (a second kernel merges).  The
 * library allocates and frees nothing.  A launch whose workspace
 * (fat_paged_decode_workspace_bytes of its batch * q_len rows) exceeds the
 * maximum returns FAT_E_INVALID.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (e.g. on two streams) race.  The
 * current HIP device must be the one `stream` belongs to (FAT_E_INVALID
 * otherwise).  The first call on a device looks up the array's address
 * (hipGetSymbolAddress); make it before capturing the call in a HIP graph,
 * as a warm-up launch before capture does.  Replays of a captured call reuse
 * the same array. */
#define FAT_DECODE_NOALLOC_MAX_WORKSPACE ((size_t)32 << 20)
int fat_paged_decode_noalloc(const fat_decode_args* args, void* stream);

/* Upper bound on the optional fat_prefill_varlen workspace of any launch
 * with these K/V sizes (used by bf16 only). */
size_t fat_prefill_workspace_bytes(int32_t total_k, int32_t num_kv_heads,
                                   int32_t head_dim);

/* Bytes of workspace the launch described by `args` would use: 0 when it
 * runs without one (fp16, short sequences, the small-grid kernels).  Reads
 * only the sizes, dtype, causal and kernel fields; no device access, so a
 * caller can size the buffer before any allocation or graph capture.
 * No reference counterpart: the reference's prefill allocates nothing
 * besides its output (flashattn_tile/kernels/prefill.py:295). */
size_t fat_prefill_varlen_workspace_bytes(const fat_prefill_args* args);

/* Enqueue varlen prefill on `stream`.
 * Replaces flashattn_tile/kernels/prefill.py:236-326 (see file header). */
int fat_prefill_varlen(const fat_prefill_args* args, void* stream);

/* Bytes of workspace the paged launch described by `args` would use (its
 * packed K/V copies and, for bf16, the V pre-pass): 0 when it runs on the
 * paged kernels.  Reads only sizes, dtype, causal and kernel; no device
 * access.  No reference counterpart (see fat_prefill_paged). */
size_t fat_prefill_paged_workspace_bytes(const fat_prefill_paged_args* args);

/* Enqueue paged (chunked) prefill on `stream`.  Extends
 * flashattn_tile/kernels/prefill.py:236-326 to K/V read through the page
 * table (the reference has no counterpart; its backend needs packed K/V,
 * flashattn_tile/backend.py:158-162). */
int fat_prefill_paged(const fat_prefill_paged_args* args, void* stream);

/* Enqueue the quantisation of one paged K or V tensor on `stream`.
 * Replaces flashattn_tile/quant.py:84-142 (quantize_kv_pages). */
int fat_quantize_pages(const fat_quantize_args* args, void* stream);

/* Enqueue a one-token-per-sequence append on `stream`.
 * Replaces flashattn_tile/paging.py:172-210 (append_tokens). */
int fat_append_kv(const fat_append_args* args, void* stream);

/*
 * The numbers a paged-cache validation checks, in one launch.
 *   seq_lens   int32 [batch]
 *   page_table int32 [batch, max_pages] (row stride page_table_stride >= max_pages)
 *   out        int64 [5], device memory: min(seq_lens), max(seq_lens), the
 *              min and max of page_table[b, c] over every row b and column
 *              c < min(ceil(max(seq_lens) / page_size), max_pages) (INT32_MAX
 *              and INT32_MIN when no column is used), and
 *              sum_b ceil(max(seq_lens[b], 0) / page_size).
 */
typedef struct fat_cache_stats_args {
  const int32_t* seq_lens;
  const int32_t* page_table;
  int64_t page_table_stride;
  int32_t batch;
  int32_t max_pages;
  int32_t page_size;
  int64_t* out;
} fat_cache_stats_args;

/* Enqueue the reductions of flashattn_tile/paging.py:84-130 (validate_cache:
 * seq_lens range, used page-table range) and the page count the decode
 * partition heuristic needs on `stream`; the caller copies `out` back and
 * checks it (one device-to-host copy per validation). */
int fat_cache_stats(const fat_cache_stats_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAT_ABI_H */
