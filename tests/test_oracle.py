"""Pin the fp32 oracle (oracle/reference.py) before trusting it.

Every check is independent of the oracle's own formula: a pure-Python loop
on tiny inputs, torch's SDPA math routine, closed forms, the reference's
known-answer tests, invariants, and mutants of the oracle (a dropped scale,
a wrong GQA mapping, an off-by-one causal mask, a wrong merge weight) that
the checks must reject.
"""

from __future__ import annotations

import math
import random

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R


def _brute(q, k, v, cu_q, cu_k, causal, scale):
    """Pure-Python attention (lists of floats), one query row at a time."""
    out = torch.zeros(q.shape, dtype=torch.float64)
    heads, kv_heads, dim = q.shape[1], k.shape[1], q.shape[2]
    group = heads // kv_heads
    for b in range(len(cu_q) - 1):
        q_len, kv_len = cu_q[b + 1] - cu_q[b], cu_k[b + 1] - cu_k[b]
        for i in range(q_len):
            for h in range(heads):
                kh = h // group
                visible = [j for j in range(kv_len) if not causal or j <= i + kv_len - q_len]
                s = []
                for j in visible:
                    acc = 0.0
                    for d in range(dim):
                        acc += float(q[cu_q[b] + i, h, d]) * float(k[cu_k[b] + j, kh, d])
                    s.append(acc * scale)
                mx = max(s)
                e = [math.exp(x - mx) for x in s]
                tot = sum(e)
                for d in range(dim):
                    out[cu_q[b] + i, h, d] = sum(e[n] * float(v[cu_k[b] + j, kh, d])
                                                 for n, j in enumerate(visible)) / tot
    return out


CASES = [
    # lens_q, lens_k, heads, kv_heads, dim
    ([1, 3, 5], [1, 3, 5], 2, 2, 4),
    ([2, 4], [3, 6], 4, 2, 3),
    ([5], [5], 4, 1, 4),
    ([1, 1, 1], [4, 1, 7], 6, 3, 2),
]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_varlen_matches_brute_force(case, causal):
    lq, lk, h, hk, d = CASES[case]
    g = torch.Generator().manual_seed(100 + case)
    q = torch.randn(sum(lq), h, d, generator=g)
    k = torch.randn(sum(lk), hk, d, generator=g)
    v = torch.randn(sum(lk), hk, d, generator=g)
    cu_q = [0]
    cu_k = [0]
    for a, b in zip(lq, lk):
        cu_q.append(cu_q[-1] + a)
        cu_k.append(cu_k[-1] + b)
    scale = 0.7
    out = R.ref_attention_varlen(q, k, v, cu_q, cu_k, causal=causal, softmax_scale=scale)
    ref = _brute(q, k, v, cu_q, cu_k, causal, scale)
    torch.testing.assert_close(out.double(), ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (8, 2), (8, 1)])
def test_varlen_matches_sdpa_math(causal, heads, kv_heads):
    """torch's SDPA math routine, GQA-expanded, one sequence at a time."""
    g = torch.Generator().manual_seed(7)
    lens = [1, 9, 33]
    d = 32
    q = torch.randn(sum(lens), heads, d, generator=g)
    k = torch.randn(sum(lens), kv_heads, d, generator=g)
    v = torch.randn(sum(lens), kv_heads, d, generator=g)
    cu = [0, 1, 10, 43]
    out = R.ref_attention_varlen(q, k, v, cu, cu, causal=causal)
    grp = heads // kv_heads
    for b in range(3):
        sl = slice(cu[b], cu[b + 1])
        qq = q[sl].transpose(0, 1).unsqueeze(0)
        kk = k[sl].repeat_interleave(grp, dim=1).transpose(0, 1).unsqueeze(0)
        vv = v[sl].repeat_interleave(grp, dim=1).transpose(0, 1).unsqueeze(0)
        with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
            ref = F.scaled_dot_product_attention(qq, kk, vv, is_causal=causal)
        torch.testing.assert_close(out[sl], ref[0].transpose(0, 1), atol=2e-6, rtol=2e-6)


def test_closed_forms():
    g = torch.Generator().manual_seed(3)
    # q = 0: uniform weights -> mean of the visible values (causal: prefix means).
    L, H, D = 6, 2, 5
    q = torch.zeros(L, H, D)
    k = torch.randn(L, H, D, generator=g)
    v = torch.randn(L, H, D, generator=g)
    out = R.ref_attention_varlen(q, k, v, [0, L], [0, L], causal=True)
    prefix_mean = torch.cumsum(v, 0) / torch.arange(1, L + 1).view(L, 1, 1)
    torch.testing.assert_close(out, prefix_mean, atol=1e-6, rtol=1e-6)
    out_nc = R.ref_attention_varlen(q, k, v, [0, L], [0, L], causal=False)
    torch.testing.assert_close(out_nc, v.mean(0, keepdim=True).expand(L, H, D), atol=1e-6, rtol=1e-6)
    # First causal row sees only key 0 -> exactly v[0], whatever q is.
    q2 = torch.randn(L, H, D, generator=g) * 10
    out2 = R.ref_attention_varlen(q2, k, v, [0, L], [0, L], causal=True)
    torch.testing.assert_close(out2[0], v[0], atol=0, rtol=0)
    # A decode query sees every key (reference test_reference.py:63-72).
    out3 = R.ref_attention_varlen(q2[:1], k, v, [0, 1], [0, L], causal=True)
    s = torch.einsum("hd,lhd->hl", q2[0], k) * D ** -0.5
    p = torch.softmax(s, -1)
    torch.testing.assert_close(out3[0], torch.einsum("hl,lhd->hd", p, v), atol=1e-6, rtol=1e-6)


def test_gqa_head_mapping_kat():
    """Reference KAT (tests/test_paging.py:116-136): heads 4 / kv 2 with
    V = 1 on kv head 0 and 2 on kv head 1 -> outputs [1, 1, 2, 2]."""
    L, D = 9, 8
    k = torch.zeros(L, 2, D)
    v = torch.zeros(L, 2, D)
    v[:, 0] = 1.0
    v[:, 1] = 2.0
    q = torch.zeros(1, 4, D)
    out = R.ref_attention_varlen(q, k, v, [0, 1], [0, L], causal=True)
    torch.testing.assert_close(out[0, :, 0], torch.tensor([1.0, 1.0, 2.0, 2.0]), atol=1e-6, rtol=0)


def _paged_inputs(seed=5, lens=(5, 17, 1, 32), P=4, hk=2, h=4, d=8):
    g = torch.Generator().manual_seed(seed)
    pages = sum(math.ceil(n / P) for n in lens) + 2
    kc = torch.randn(pages, P, hk, d, generator=g)
    vc = torch.randn(pages, P, hk, d, generator=g)
    perm = torch.randperm(pages, generator=g)
    maxp = max(math.ceil(n / P) for n in lens)
    table = torch.zeros(len(lens), maxp, dtype=torch.int32)
    at = 0
    for b, n in enumerate(lens):
        m = math.ceil(n / P)
        table[b, :m] = perm[at:at + m].int()
        at += m
    q = torch.randn(len(lens), h, d, generator=g)
    return q, kc, vc, table, torch.tensor(lens, dtype=torch.int32)


def test_paged_equals_varlen_on_gather_and_is_permutation_invariant():
    q, kc, vc, table, lens = _paged_inputs()
    out = R.ref_attention_paged(q, kc, vc, table, lens)
    ks, vs = R.gather_pages(kc, vc, table, lens)
    for b in range(q.shape[0]):
        n = int(lens[b])
        exp = R.ref_attention_varlen(q[b:b + 1], ks[b], vs[b], [0, 1], [0, n])
        torch.testing.assert_close(out[b:b + 1], exp, atol=0, rtol=0)
        # contiguous restatement: page p of the sequence holds tokens p*P..p*P+P-1
        P = kc.shape[1]
        direct = torch.stack([kc[int(table[b, t // P]), t % P] for t in range(n)])
        torch.testing.assert_close(ks[b], direct, atol=0, rtol=0)
    # Permute the physical pool and remap the table: same result.
    g = torch.Generator().manual_seed(9)
    perm = torch.randperm(kc.shape[0], generator=g)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(kc.shape[0])
    out2 = R.ref_attention_paged(q, kc[perm], vc[perm], inv[table.long()].int(), lens)
    torch.testing.assert_close(out2, out, atol=0, rtol=0)


def test_dense_wrapper_matches_varlen():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(2, 4, 6, 16, generator=g)
    k = torch.randn(2, 2, 6, 16, generator=g)
    v = torch.randn(2, 2, 6, 16, generator=g)
    out = R.ref_attention_dense(q, k, v, causal=True)
    for b in range(2):
        exp = R.ref_attention_varlen(q[b].transpose(0, 1).contiguous(), k[b].transpose(0, 1).contiguous(),
                                     v[b].transpose(0, 1).contiguous(), [0, 6], [0, 6])
        torch.testing.assert_close(out[b], exp.transpose(0, 1), atol=0, rtol=0)


def test_lse_merge_any_partition_equals_unsplit():
    g = torch.Generator().manual_seed(11)
    L, H, D = 37, 3, 8
    q = torch.randn(H, D, generator=g)
    k = torch.randn(L, H, D, generator=g)
    v = torch.randn(L, H, D, generator=g)
    whole = R.lse_merge(R.lse_partials(q, k, v, [(0, L)], 0.3))
    rnd = random.Random(0)
    for _ in range(5):
        cuts = sorted(rnd.sample(range(1, L), 4))
        bounds = list(zip([0] + cuts, cuts + [L])) + [(L, L), (5, 5)]  # two empty partitions
        merged = R.lse_merge(R.lse_partials(q, k, v, bounds, 0.3))
        torch.testing.assert_close(merged, whole, atol=1e-6, rtol=1e-6)
    s = torch.einsum("hd,lhd->hl", q, k) * 0.3
    direct = torch.einsum("hl,lhd->hd", torch.softmax(s, -1), v)
    torch.testing.assert_close(whole, direct, atol=1e-6, rtol=1e-6)


def test_validation_messages():
    q = torch.randn(4, 1, 8)
    k = torch.randn(2, 1, 8)
    with pytest.raises(ValueError, match="kv_len >= q_len"):
        R.ref_attention_varlen(q, k, k, [0, 4], [0, 2], causal=True)
    with pytest.raises(ValueError, match="must start at 0"):
        R.ref_attention_varlen(q, q, q, [1, 4], [0, 4])
    with pytest.raises(ValueError, match="non-decreasing"):
        R.ref_attention_varlen(q, q, q, [0, 4, 2], [0, 2, 4])
    with pytest.raises(ValueError, match="ends at"):
        R.ref_attention_varlen(q, q, q, [0, 3], [0, 4])
    with pytest.raises(ValueError, match="divisible"):
        R.ref_attention_varlen(torch.randn(3, 5, 8), torch.randn(3, 2, 8), torch.randn(3, 2, 8), [0, 3], [0, 3])
    with pytest.raises(ValueError, match="at least one cached token"):
        R.ref_attention_paged(torch.randn(1, 2, 4), torch.randn(2, 4, 1, 4), torch.randn(2, 4, 1, 4),
                              torch.zeros(1, 1, dtype=torch.int32), torch.zeros(1, dtype=torch.int32))


def test_output_dtype_and_fp32_view():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(16, 4, 32, generator=g)
    k = torch.randn(16, 2, 32, generator=g)
    v = torch.randn(16, 2, 32, generator=g)
    cu = [0, 5, 16]
    for dt in (torch.float16, torch.bfloat16):
        out = R.ref_attention_varlen(q.to(dt), k.to(dt), v.to(dt), cu, cu)
        r32 = R.ref_attention_varlen(q.to(dt), k.to(dt), v.to(dt), cu, cu, return_fp32=True)
        assert out.dtype == dt and r32.dtype == torch.float32
        torch.testing.assert_close(out, r32.to(dt), atol=0, rtol=0)


# ---------------------------------------------------------------------------
# Planted mistakes: each mutant oracle must be rejected by the checks above.
# ---------------------------------------------------------------------------
def _mutant_attend(kind, orig):
    def attend(qb, kb, vb, group, causal, scale):
        if kind == "gqa":
            kb = kb.float().repeat(1, group, 1)  # h % Hkv instead of h // group
            vb = vb.float().repeat(1, group, 1)
            return orig(qb, kb, vb, 1, causal, scale)
        if kind == "scale":
            return orig(qb, kb, vb, group, causal, 1.0)
        if kind == "causal":
            q_len, kv_len = qb.shape[0], kb.shape[0]
            kf = kb.float().repeat_interleave(group, dim=1)
            vf = vb.float().repeat_interleave(group, dim=1)
            s = torch.einsum("qhd,khd->hqk", qb.float(), kf) * scale
            if causal:
                rows = torch.arange(q_len).unsqueeze(1) + kv_len - q_len
                bad = torch.arange(kv_len).unsqueeze(0) > rows - 1  # j < i visible only
                bad[:, 0] = False
                s = s.masked_fill(bad.unsqueeze(0), float("-inf"))
            return torch.einsum("hqk,khd->qhd", torch.softmax(s, -1), vf)
        raise AssertionError(kind)
    return attend


@pytest.mark.parametrize("kind", ["gqa", "scale", "causal"])
def test_planted_mistakes_are_caught(kind, monkeypatch):
    monkeypatch.setattr(R, "_attend_one", _mutant_attend(kind, R._attend_one))
    caught = False
    try:
        if kind == "gqa":
            test_gqa_head_mapping_kat()
        elif kind == "scale":
            test_varlen_matches_sdpa_math(False, 8, 2)
        else:
            test_varlen_matches_brute_force(0, True)
    except AssertionError:
        caught = True
    assert caught, f"mutant '{kind}' passed the oracle checks"


def test_planted_merge_mistake_is_caught():
    def bad_merge(parts):
        m_all = torch.stack([m for _, m, _ in parts])
        m_star = m_all.max(dim=0).values
        num = sum(acc * torch.exp(m - m_star)[:, None] for acc, m, _ in parts)
        den = sum(l for _, _, l in parts)  # forgot the exp(m - m*) weight
        return num / den[:, None]

    g = torch.Generator().manual_seed(12)
    q, k, v = torch.randn(2, 4, generator=g), torch.randn(20, 2, 4, generator=g), torch.randn(20, 2, 4, generator=g)
    parts = R.lse_partials(q, k, v, [(0, 7), (7, 20)], 1.0)
    whole = R.lse_merge(R.lse_partials(q, k, v, [(0, 20)], 1.0))
    assert not torch.allclose(bad_merge(parts), whole, atol=1e-4)


def _pool_from_packed(k, v, lens, page_size, perm_seed=None):
    """A paged pool holding packed per-sequence K/V, pages optionally permuted."""
    import math as _m

    pages = [_m.ceil(n / page_size) for n in lens]
    num_pages = sum(pages)
    kc = torch.zeros(num_pages, page_size, k.shape[1], k.shape[2], dtype=k.dtype)
    vc = torch.zeros_like(kc)
    order = torch.arange(num_pages)
    if perm_seed is not None:
        order = torch.randperm(num_pages, generator=torch.Generator().manual_seed(perm_seed))
    table = torch.zeros(len(lens), max(pages), dtype=torch.int32)
    at_page, at_tok = 0, 0
    for b, n in enumerate(lens):
        for i in range(pages[b]):
            phys = int(order[at_page + i])
            table[b, i] = phys
            lo = at_tok + i * page_size
            hi = min(at_tok + n, lo + page_size)
            kc[phys, : hi - lo] = k[lo:hi]
            vc[phys, : hi - lo] = v[lo:hi]
        at_page += pages[b]
        at_tok += n
    return kc, vc, table, torch.tensor(lens, dtype=torch.int32)


def test_paged_prefill_oracle_pins():
    from oracle.reference import ref_attention_paged, ref_attention_paged_prefill, ref_attention_varlen

    g = torch.Generator().manual_seed(31)
    lens_k, lens_q = [5, 9, 1, 12], [2, 9, 1, 3]
    h, hk, d, P = 4, 2, 8, 4
    k = torch.randn(sum(lens_k), hk, d, generator=g)
    v = torch.randn(sum(lens_k), hk, d, generator=g)
    q = torch.randn(sum(lens_q), h, d, generator=g)
    cu_q = [0]
    for n in lens_q:
        cu_q.append(cu_q[-1] + n)
    cu_k = [0]
    for n in lens_k:
        cu_k.append(cu_k[-1] + n)
    kc, vc, table, sl = _pool_from_packed(k, v, lens_k, P)
    # 1. a pool holding the packed K/V in order: the varlen result itself
    got = ref_attention_paged_prefill(q, kc, vc, table, sl, cu_q, causal=True)
    assert torch.equal(got, ref_attention_varlen(q, k, v, cu_q, cu_k, causal=True))
    # 2. page-table permutation invariance
    kc2, vc2, table2, _ = _pool_from_packed(k, v, lens_k, P, perm_seed=4)
    assert torch.equal(ref_attention_paged_prefill(q, kc2, vc2, table2, sl, cu_q, causal=True), got)
    # 3. one query per sequence: the decode oracle
    q1 = torch.randn(len(lens_k), h, d, generator=g)
    cu1 = list(range(len(lens_k) + 1))
    assert torch.equal(ref_attention_paged_prefill(q1, kc, vc, table, sl, cu1, causal=True),
                       ref_attention_paged(q1, kc, vc, table, sl, causal=True))
    # 4. chunking identity: a 12-token causal prompt as chunks [0, 7) and
    # [7, 12) (kv lengths 7 and 12) gives the one-shot rows.  A top-left
    # causal convention (shift 0) would fail this.
    L = 12
    qf = torch.randn(L, h, d, generator=g)
    kf = torch.randn(L, hk, d, generator=g)
    vf = torch.randn(L, hk, d, generator=g)
    kcf, vcf, tf, _ = _pool_from_packed(kf, vf, [L], P)
    one = ref_attention_paged_prefill(qf, kcf, vcf, tf, torch.tensor([L], dtype=torch.int32), [0, L])
    c1 = ref_attention_paged_prefill(qf[:7], kcf, vcf, tf, torch.tensor([7], dtype=torch.int32), [0, 7])
    c2 = ref_attention_paged_prefill(qf[7:], kcf, vcf, tf, torch.tensor([L], dtype=torch.int32), [0, 5])
    torch.testing.assert_close(torch.cat([c1, c2]), one, rtol=0, atol=1e-6)
    wrong = ref_attention_varlen(qf[7:], kf[:5], vf[:5], [0, 5], [0, 5], causal=True)  # shift dropped
    assert (wrong - one[7:]).abs().max() > 1e-2
