"""GPU parity of the paged (chunked) prefill, ``fat_prefill_paged``.

Each sequence's queries (a chunk of q_len tokens) attend to the first
seq_lens[b] keys of a paged cache whose pages are scattered by a seeded
permutation and whose slots past each sequence end are poisoned (K = 30,
V = 500).  The oracle is ``ref_attention_paged_prefill`` (gather through the
table, then the fp32 varlen restatement of flashattn_tile/reference.py); the
tolerance is the north star's 2e-3 on the kernel's result before its final
rounding (tests/_parity.py).  Every shape runs on both prefill kernels.
"""

from __future__ import annotations

import pytest
import torch

from _parity import assert_parity, force_prefill_knobs, make_paged
from flashattntile_amd import PagedKVCache
from flashattntile_amd.kernels.prefill import paged_prefill_attention, prefill_attention
from flashattntile_amd.paging import gather_contiguous
from oracle.reference import ref_attention_paged_prefill, ref_attention_varlen

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(params=["auto", "pingpong", "4wave", "4wave_split"])
def kernel(request, monkeypatch):
    if request.param != "auto":
        force_prefill_knobs(monkeypatch, kernel=request.param)
    return request.param


def _case(lens_k, lens_q, h, hk, d, P, dtype, seed):
    k, v, pt, sl = make_paged(lens_k, hk, d, P, dtype, seed=seed, device=DEV)
    g = torch.Generator().manual_seed(seed + 100)
    q = torch.randn(sum(lens_q), h, d, generator=g).to(dtype).to(DEV)
    cu = torch.tensor([0] + torch.cumsum(torch.tensor(lens_q), 0).tolist(), dtype=torch.int32, device=DEV)
    return q, PagedKVCache(k, v, pt, sl, P), cu


def _ref32(q, cache, cu, causal, scale=None):
    return ref_attention_paged_prefill(q.cpu(), cache.k_cache.cpu(), cache.v_cache.cpu(), cache.page_table.cpu(),
                                       cache.seq_lens.cpu(), cu.cpu(), causal=causal, softmax_scale=scale,
                                       return_fp32=True)


# chunks: (kv_len, q_len) per sequence -- a whole prompt, a chunk after a
# prefix, single-token chunks (multi-sequence decode), a chunk crossing pages
CHUNKS = [(1000, 1000), (300, 77), (129, 1), (64, 64), (517, 200), (5, 3)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("h,hk", [(8, 8), (8, 2), (32, 8), (8, 1)])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_prefill_matches_oracle(dtype, d, h, hk, causal, kernel):
    label = f"paged prefill {kernel} {dtype} D{d} H{h}/{hk} causal={causal}"
    print(label, flush=True)
    lens_k = [c[0] for c in CHUNKS]
    lens_q = [c[1] for c in CHUNKS]
    q, cache, cu = _case(lens_k, lens_q, h, hk, d, 16, dtype, seed=d + h + hk)
    out = paged_prefill_attention(q, cache, cu, max(lens_q), causal=causal)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == dtype
    assert_parity(out, _ref32(q, cache, cu, causal), label=label)


# (kv_len, q_len): sequences with no new tokens this step (q_len = 0), with
# cached keys or none, around sequences that prefill a chunk.
IDLE_CHUNKS = [(1000, 0), (300, 77), (129, 0), (0, 0), (64, 64), (517, 0), (5, 3), (40, 0)]


@pytest.mark.parametrize("P", [1, 16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_prefill_batch_with_idle_sequences(dtype, causal, P, kernel):
    """A paged batch in which some sequences have no new tokens: parity, and
    the working rows bit-identical, on a forced kernel, to a batch of only those."""
    label = f"paged prefill {kernel} {dtype} P{P} idle sequences causal={causal}"
    print(label, flush=True)
    lens_k = [c[0] for c in IDLE_CHUNKS]
    lens_q = [c[1] for c in IDLE_CHUNKS]
    q, cache, cu = _case(lens_k, lens_q, 16, 4, 128, P, dtype, seed=53 + P)
    out = paged_prefill_attention(q, cache, cu, max(lens_q), causal=causal)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache, cu, causal), label=label)
    if kernel == "auto":  # the smaller batch may get another kernel
        return
    keep = [i for i, n in enumerate(lens_q) if n > 0]
    sub = PagedKVCache(cache.k_cache, cache.v_cache, cache.page_table[keep].contiguous(),
                       cache.seq_lens[keep].contiguous(), P)
    cu2 = torch.tensor([0] + torch.cumsum(torch.tensor([lens_q[i] for i in keep]), 0).tolist(), dtype=torch.int32,
                       device=DEV)
    out2 = paged_prefill_attention(q, sub, cu2, max(lens_q), causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), label


@pytest.mark.parametrize("P", [4, 16, 64])
@pytest.mark.parametrize("d", [32, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_prefill_head_dims_32_and_256(dtype, d, P):
    """head_dim 32 and 256 through the page table, with pages below, at and
    above the rows of one 16-byte-per-lane load (64 at D32, 8 at D256), on
    the library's kernel choice."""
    label = f"paged prefill {dtype} D{d} P{P}"
    print(label, flush=True)
    lens_k = [c[0] for c in CHUNKS]
    lens_q = [c[1] for c in CHUNKS]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, d, P, dtype, seed=d + P)
    out = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache, cu, True), label=label)


@pytest.mark.parametrize("P", [1, 4, 16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_prefill_page_sizes(P, dtype, kernel):
    label = f"paged prefill {kernel} P{P} {dtype}"
    print(label, flush=True)
    lens_k, lens_q = [333, 64, 1, 200], [100, 64, 1, 7]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, 128, P, dtype, seed=P)
    out = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True, softmax_scale=0.06)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache, cu, True, scale=0.06), label=label)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_prefill_equals_packed_prefill(dtype, kernel):
    """The same keys, paged or packed: both prefill kernels agree bit for bit
    (the paged path changes only where K/V rows are read from)."""
    lens = [700, 129, 1, 64]
    q, cache, cu = _case(lens, lens, 16, 4, 128, 16, dtype, seed=5)
    k, v = gather_contiguous(cache)
    pk = torch.cat([k[b, :n] for b, n in enumerate(lens)])
    pv = torch.cat([v[b, :n] for b, n in enumerate(lens)])
    out_paged = paged_prefill_attention(q, cache, cu, max(lens), causal=True)
    out_packed = prefill_attention(q, pk, pv, cu, cu, max(lens), max(lens), causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out_paged, out_packed)


# (kv_len, q_len): long chunks, a chunk after a prefix, sequences without
# new tokens (with and without cached keys).
STAGED = [(2100, 2100), (1500, 600), (0, 0), (700, 0), (2600, 2047)]


@pytest.mark.parametrize("P", [1, 16, 256])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_staged_paged_prefill_matches_oracle(dtype, causal, P, monkeypatch):
    """Forced onto the wide kernel, a paged launch copies the used K/V rows
    (through the permuted table; slots past each sequence end are poisoned)
    into its workspace, computes the sequences' offsets on the device, and
    runs the packed wide kernel on the copies (bf16: after the V pre-pass)."""
    from flashattntile_amd import _hip

    force_prefill_knobs(monkeypatch, kernel="wide")
    label = f"staged paged prefill {dtype} P{P} causal={causal}"
    print(label, flush=True)
    lens_k = [c[0] for c in STAGED]
    lens_q = [c[1] for c in STAGED]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, 128, P, dtype, seed=P + 40)
    a = _hip.prefill_paged_args(q, cache.k_cache, cache.v_cache, cache.page_table, cache.seq_lens, cu, q,
                                P, max(lens_q), causal, 128 ** -0.5, kernel=_hip.KERNEL_PREFILL_WIDE)
    assert _hip.prefill_paged_workspace_bytes(a) > 0
    out = paged_prefill_attention(q, cache, cu, max(lens_q), causal=causal)
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache, cu, causal), label=label)


def test_staged_paged_prefill_agrees_with_the_paged_kernel():
    """The same causal bf16 launch staged (wide kernel on the copies) and on
    the paged ping-pong kernel: both within the tolerance of the oracle, and
    within twice that of each other."""
    lens_k, lens_q = [3000, 2200], [3000, 2100]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, 128, 16, torch.bfloat16, seed=5)
    staged = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True, config={"kernel": "wide"})
    paged = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True, config={"kernel": "pingpong"})
    torch.cuda.synchronize()
    ref = _ref32(q, cache, cu, True)
    assert_parity(staged, ref, label="staged bf16")
    assert_parity(paged, ref, label="paged bf16")
    assert_parity(staged, paged.float(), tol=4e-3, label="staged vs paged")


def test_paged_prefill_32k_sequence_first_and_last_rows():
    """One causal fp16 sequence of 32768 tokens (2048 pages of 16, permuted)
    read through the page table: the first and last 256 rows of KV heads 0
    and 7 against the fp32 oracle on the gathered keys (the first rows see
    the first 256 tokens only; the last rows, bottom-right aligned, all)."""
    L, n = 32768, 256
    print("paged prefill 32k", flush=True)
    q, cache, cu = _case([L], [L], 32, 8, 128, 16, torch.float16, seed=32)
    out = paged_prefill_attention(q, cache, cu, L, causal=True)
    torch.cuda.synchronize()
    k, v = gather_contiguous(cache)
    k, v = k[0, :L], v[0, :L]
    cu_n = torch.tensor([0, n], dtype=torch.int32)
    cu_l = torch.tensor([0, L], dtype=torch.int32)
    for kvh in (0, 7):
        hs = slice(4 * kvh, 4 * kvh + 4)
        kk, vv = k[:, kvh:kvh + 1].cpu().contiguous(), v[:, kvh:kvh + 1].cpu().contiguous()
        first = ref_attention_varlen(q[:n, hs].cpu().contiguous(), kk[:n].contiguous(), vv[:n].contiguous(), cu_n,
                                     cu_n, causal=True, return_fp32=True)
        last = ref_attention_varlen(q[L - n:, hs].cpu().contiguous(), kk, vv, cu_n, cu_l, causal=True,
                                    return_fp32=True)
        assert_parity(out[:n, hs], first, label=f"paged prefill 32k kv{kvh} first rows")
        assert_parity(out[L - n:, hs], last, label=f"paged prefill 32k kv{kvh} last rows")


def test_paged_prefill_chunked_equals_one_shot(kernel):
    """A prompt prefilled in three chunks through the cache gives the rows of
    the one-shot causal prefill (bottom-right alignment)."""
    L, P, h, hk, d = 900, 16, 8, 2, 128
    q, cache, cu = _case([L], [L], h, hk, d, P, torch.float16, seed=9)
    full = paged_prefill_attention(q, cache, cu, L, causal=True)
    parts = []
    for lo, hi in ((0, 300), (300, 301), (301, L)):
        chunk = PagedKVCache(cache.k_cache, cache.v_cache, cache.page_table,
                             torch.tensor([hi], dtype=torch.int32, device=DEV), P)
        ccu = torch.tensor([0, hi - lo], dtype=torch.int32, device=DEV)
        parts.append(paged_prefill_attention(q[lo:hi].contiguous(), chunk, ccu, hi - lo, causal=True))
    torch.cuda.synchronize()
    got = torch.cat(parts)
    # both sides are kernel outputs, each within 2e-3 of the oracle
    assert_parity(got, full.float(), tol=4e-3, label="chunked vs one-shot")
    assert_parity(got, _ref32(q, cache, cu, True), label="chunked vs oracle")


def test_paged_prefill_validation():
    lens_k, lens_q = [10, 20], [4, 25]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, 64, 16, torch.float16, seed=1)
    with pytest.raises(ValueError, match="kv_len >= q_len"):
        paged_prefill_attention(q, cache, cu, 25, causal=True)
    out = paged_prefill_attention(q, cache, cu, 25, causal=False)  # allowed without causal masking
    torch.cuda.synchronize()
    assert_parity(out, _ref32(q, cache, cu, False), label="non-causal q_len > kv_len")
    with pytest.raises(ValueError, match="max_seqlen_q"):
        paged_prefill_attention(q, cache, cu, 5, causal=False)
    bad = PagedKVCache(cache.k_cache, cache.v_cache, cache.page_table.clone(), cache.seq_lens, 16)
    bad.page_table[1, 0] = cache.num_pages
    with pytest.raises(AssertionError, match="references page"):
        paged_prefill_attention(q, bad, cu, 25, causal=False)
    with pytest.raises(ValueError, match="batch \\+ 1"):
        paged_prefill_attention(q, cache, cu[:2], 25, causal=False)


@pytest.mark.parametrize("P", [16, 32, 64])
def test_paged_prefill_row_modes_agree(P):
    """Pages of >= 16 rows take the wave-uniform addressing (32-bit pool
    offsets for a pool under 2 GiB); forcing 64-bit row addresses or the
    per-lane addressing on the same inputs must give identical bits."""
    print(f"paged P{P} row modes", flush=True)
    lens_k, lens_q = [900, 70, 129], [300, 70, 1]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, 128, P, torch.bfloat16, seed=P + 1)
    uni = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True)
    wide = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True, config={"rows": "wide"})
    lane = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True, config={"rows": "lane"})
    torch.cuda.synchronize()
    assert torch.equal(uni, lane) and torch.equal(uni, wide)
    assert_parity(uni, _ref32(q, cache, cu, True), label=f"paged P{P} uniform rows")


def test_paged_prefill_ignores_nan_past_seq_len(kernel):
    """Slots past each sequence's end hold NaN: the kernel must never let them
    into the result (the wave-uniform path zeroes those rows before LDS)."""
    lens_k, lens_q = [100, 37, 64], [100, 5, 64]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, 128, 32, torch.float16, seed=3)
    for b, n in enumerate(lens_k):
        pages = (n + 31) // 32
        last = int(cache.page_table[b, pages - 1])
        used = n - (pages - 1) * 32
        if used < 32:
            cache.k_cache[last, used:] = float("nan")
            cache.v_cache[last, used:] = float("nan")
    out = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert_parity(out, _ref32(q, cache, cu, True), label="NaN past seq_len")


def test_prefill_paged_op_and_backend_route():
    """The extension op and the backend's paged-prefill route run the same
    kernel as the function (also under torch.compile(fullgraph=True))."""
    from flashattntile_amd.backend import AttentionMetadata, FlashAttnTileBackend

    lens_k, lens_q = [300, 77], [20, 77]
    q, cache, cu = _case(lens_k, lens_q, 8, 2, 128, 16, torch.float16, seed=77)
    want = paged_prefill_attention(q, cache, cu, max(lens_q), causal=True, softmax_scale=0.09)

    def op(x):
        return torch.ops.flashattn_tile.prefill_paged(x, cache.k_cache, cache.v_cache, cache.page_table,
                                                      cache.seq_lens, cu, max(lens_q), 16, True, 0.09)

    got = op(q)
    compiled = torch.compile(op, fullgraph=True)(q)
    backend = FlashAttnTileBackend(num_heads=8, num_kv_heads=2, head_dim=128, page_size=16)
    routed = backend.forward(q, cache, AttentionMetadata(is_prefill=True, paged_prefill=True, cu_seqlens_q=cu,
                                                         max_seqlen_q=max(lens_q), softmax_scale=0.09))
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(compiled, want) and torch.equal(routed, want)


@pytest.mark.parametrize("P", [4, 16])
@pytest.mark.parametrize("kern", [None, "pingpong", "4wave", "4wave_split"])
def test_paged_prefill_output_rows_only_8_byte_aligned(kern, P):
    """Paged prefill into output rows that start 8 bytes past a 16-byte
    boundary (base offset 4 elements, head stride 68): each row leaves in
    8-byte pieces and the gaps between heads stay untouched."""
    from flashattntile_amd.kernels.prefill import paged_prefill_launch

    print(f"paged prefill 8-byte-aligned out {kern or 'auto'} P{P}", flush=True)
    q, cache, cu = _case([300, 517, 64], [300, 200, 64], 8, 2, 64, P, torch.float16, seed=9)
    big = torch.zeros(q.shape[0], 8, 68, dtype=q.dtype, device=DEV)
    out = big[:, :, 4:]
    assert out.data_ptr() % 16 == 8
    paged_prefill_launch(q, cache, cu, 300, True, 64 ** -0.5, out=out, kernel=kern)
    torch.cuda.synchronize()
    assert torch.all(big[:, :, :4] == 0)
    assert_parity(out, _ref32(q, cache, cu, True, scale=64 ** -0.5), label=f"paged 8-byte-aligned out {kern} P{P}")
