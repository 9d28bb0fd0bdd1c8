"""Analytic work formulas (reference KATs, tests/test_autotune.py:13-50) and
the MI355X split heuristic."""

from __future__ import annotations

import pytest

from flashattntile_amd import autotune as at


def test_flops_causal_and_noncausal():
    assert at.flops_attention(1, 4, 2, 3, causal=False) == 96
    assert at.flops_attention(1, 4, 2, 3, causal=True) == 80
    assert at.flops_attention(8, 128, 1, 4096, causal=True, batch=4) == 4 * 4 * 8 * 128 * 4096


def test_flops_varlen_sums_sequences():
    total = at.flops_attention_varlen(2, 8, [1, 4], [10, 4], causal=True)
    assert total == at.flops_attention(2, 8, 1, 10, causal=True) + at.flops_attention(2, 8, 4, 4, causal=True)
    with pytest.raises(ValueError):
        at.flops_attention_varlen(2, 8, [1], [1, 2])


def test_bytes_decode_and_prefill():
    nbytes = at.bytes_attention("decode", 8, 1, 4096, 32, 8, 128, elem_bytes=2)
    assert nbytes == 8 * 4096 * 8 * 128 * 2 * 2 + 2 * 8 * 32 * 128 * 2
    assert 3.0 < at.arithmetic_intensity(at.flops_attention(32, 128, 1, 4096, True, 8), nbytes) < 5.0
    assert at.bytes_attention("prefill", 1, 1024, 1024, 32, 8, 128, 2) == 2 * (1024 * 32 * 128 * 2) + 1024 * 8 * 128 * 4
    with pytest.raises(ValueError):
        at.bytes_attention("backward", 1, 1, 1, 1, 1, 1)
    with pytest.raises(ValueError):
        at.bytes_attention("decode", 1, 2, 4, 1, 1, 1)


def test_baseline_work_numbers():
    """The roofline numerators quoted for the BASELINE configs."""
    assert at.bytes_attention("decode", 32, 1, 4096, 32, 8, 128) == 537_395_200
    assert at.bytes_decode_paged([4096] * 32, 32, 8, 128) == 537_395_200
    assert at.flops_attention(32, 128, 8192, 8192, causal=True) == 549_822_922_752
    assert at.flops_attention(32, 128, 512, 512, causal=True) == 2_151_677_952
    q = at.bytes_decode_paged([16384] * 128, 32, 8, 128, q_elem_bytes=2, kv_elem_bytes=1, page_size=16,
                              quantized=True)
    assert q == 4_305_453_056
    assert at.bytes_decode_paged([131072], 32, 8, 128) == 536_887_296


def test_split_heuristic():
    # the measured MI355X optima (32/8 heads, D128, page 16)
    assert at.decode_split_k(32, 32, 8, 256) == 1
    assert at.decode_split_k(8, 32, 8, 256) == 4
    assert at.decode_split_k(1, 32, 8, 64) == 8
    assert at.decode_split_k(1, 32, 8, 1024) == 16
    assert at.decode_split_k(1, 32, 8, 8192) == 16  # capped
    assert at.decode_split_k(128, 32, 8, 1024) == 1
    assert at.decode_split_k(1, 32, 8, 3) == 1  # partitions of at least 8 pages


def test_partition_heuristic():
    # uniform batches: same launches as decode_split_k
    assert at.decode_partition(32, 32, 8, 256, 32 * 256) == (1, 256)
    assert at.decode_partition(8, 32, 8, 256, 8 * 256) == (4, 64)
    assert at.decode_partition(1, 32, 8, 64, 64) == (8, 8)
    # short partitions: capped at 16, pages re-spread over them
    assert at.decode_partition(1, 32, 8, 1024, 1024) == (16, 64)
    # partitions of >= 256 pages: up to 64 of them, so B1 ctx131072 fills the CUs
    assert at.decode_partition(1, 32, 8, 8192, 8192) == (32, 256)
    # skewed batch: ~4 workgroups per CU, an odd split covering the longest sequence
    split, chunk = at.decode_partition(64, 32, 8, 4096, 40019)
    c0 = -(-40019 * 8 // (4 * 256))
    s0 = -(-4096 // c0)
    assert split == (s0 + 1 if s0 % 2 == 0 else s0) and chunk == -(-4096 // split)
    assert split % 2 == 1 and split * chunk >= 4096 and split <= 64
    # the bench's 64 log-uniform lengths and 2 x 65536 + 30 x 512 (measured best at 13 and 57 partitions)
    assert at.decode_partition(64, 32, 8, 3998, 40049) == (13, 308)
    assert at.decode_partition(32, 32, 8, 4096, 9152) == (57, 72)
    # at the 64-partition cap an even split steps down (one 100000-page sequence among 15 of one page)
    assert at.decode_partition(16, 32, 8, 100000, 100015) == (63, 1588)


# ---------------------------------------------------------------------------
# gfx950 tuned-config store (schema of the reference's autotune.py:376-419)
# ---------------------------------------------------------------------------
def test_signatures():
    import torch

    # packed prefill keeps the reference's key (prefill.py:276), e.g. its
    # store's "prefill:B1_H32_Hkv8_D128_Lq512_Lk512_c1"
    assert at.prefill_signature(1, 32, 8, 128, 512, 512, True) == "B1_H32_Hkv8_D128_Lq512_Lk512_c1"
    assert at.prefill_paged_signature(2, 32, 8, 128, 16, 512, False) == "B2_H32_Hkv8_D128_P16_Lq512_c0"
    sig = at.decode_signature(32, 32, 8, 128, 16, 4096, 32 * 256, torch.float16)
    assert sig == "B32_H32_Hkv8_D128_P16_L4096_fp16"
    assert at.decode_signature(128, 32, 8, 128, 16, 16384, 128 * 1024, torch.float8_e4m3fn).endswith("_fp8")
    assert at.decode_signature(128, 32, 8, 128, 16, 16384, 128 * 1024, torch.int8).endswith("_int8")
    assert at.decode_signature(32, 32, 8, 128, 16, 4096, 32 * 256, torch.bfloat16, q_len=4).endswith("_bf16_T4")
    # one long sequence among short ones: the ragged regime of decode_partition
    assert at.decode_signature(4, 32, 8, 128, 16, 4096, 256 + 3, torch.float16).endswith("_ragged")
    assert at.is_ragged(4, 256, 259) and not at.is_ragged(4, 256, 4 * 256)


def test_store_round_trip(tmp_path, monkeypatch):
    path = tmp_path / "store.json"
    monkeypatch.delenv("FAT_TUNED_CONFIGS", raising=False)
    assert at.best_config("decode", "x", path=path) is None  # missing file = empty store
    at.initialize_store("note one", path=path)
    at.save_best("decode", "B1_sig", {"split_k": 4, "kernel": "mfma"}, {"latency_ms": 0.1}, path=path)
    data = __import__("json").loads(path.read_text())
    assert data["_meta"]["schema_version"] == 1 and data["_meta"]["arch"] == "gfx950"
    assert data["_meta"]["note"] == "note one" and "updated_utc" in data["_meta"]
    entry = data["configs"]["decode:B1_sig"]
    assert entry["kind"] == "decode" and entry["signature"] == "B1_sig" and entry["metrics"] == {"latency_ms": 0.1}
    assert at.best_config("decode", "B1_sig", path=path) == {"split_k": 4, "kernel": "mfma"}
    assert at.best_config("prefill", "B1_sig", path=path) is None
    # a second save replaces the entry and is seen by the next lookup (mtime/size-keyed cache)
    at.save_best("decode", "B1_sig", {"split_k": 16, "kernel": "valu"}, path=path)
    assert at.best_config("decode", "B1_sig", path=path) == {"split_k": 16, "kernel": "valu"}
    # the returned dict is a copy: mutating it does not change the store
    at.best_config("decode", "B1_sig", path=path)["split_k"] = 99
    assert at.best_config("decode", "B1_sig", path=path)["split_k"] == 16
    # a corrupt file reads as an empty store
    path.write_text("{not json")
    assert at.best_config("decode", "B1_sig", path=path) is None
    # FAT_TUNED_CONFIGS selects the file, "none" disables lookups
    good = tmp_path / "good.json"
    at.save_best("prefill", "P", {"kernel": "4wave"}, path=good)
    monkeypatch.setenv("FAT_TUNED_CONFIGS", str(good))
    assert at.best_config("prefill", "P") == {"kernel": "4wave"}
    monkeypatch.setenv("FAT_TUNED_CONFIGS", "none")
    assert at.best_config("prefill", "P") is None
    with pytest.raises(ValueError, match="disabled"):
        at.save_best("prefill", "P", {"kernel": "4wave"})


def test_committed_store_is_well_formed():
    import json

    data = json.loads(at.TUNED_CONFIGS_PATH.read_text())
    assert data["_meta"]["schema_version"] == 1 and data["_meta"]["arch"] == "gfx950"
    for key, entry in data["configs"].items():
        kind, sig = key.split(":", 1)
        assert entry["kind"] == kind and entry["signature"] == sig
        cfg = entry["config"]
        if kind == "decode":
            assert set(cfg) <= {"split_k", "pages_per_split", "num_warps", "kernel"}
            assert 1 <= cfg["split_k"] <= 64 and cfg.get("num_warps") in (None, 4, 8)
            assert cfg.get("kernel") in (None, "valu", "mfma")
        else:
            assert kind in ("prefill", "prefill_paged") and set(cfg) == {"kernel"}
            assert cfg["kernel"] in (None, "pingpong", "wide", "4wave", "4wave_split")


def test_config_space():
    space = at.build_config_space("decode", batch=32, num_heads=32, num_kv_heads=8, max_pages=256)
    assert space[0] == {"split_k": 1, "pages_per_split": 256, "num_warps": 4, "kernel": "valu"}  # heuristic first
    assert {c["kernel"] for c in space} == {"valu", "mfma"} and {c["num_warps"] for c in space} == {4, 8}
    assert max(c["split_k"] for c in space) == 64
    assert len({tuple(sorted(c.items())) for c in space}) == len(space)
    short = at.build_config_space("decode", batch=1, max_pages=3)
    assert max(c["split_k"] for c in short) == 3  # at least one page per partition
    multi = at.build_config_space("decode", batch=32, max_pages=256, q_len=4)
    assert {c["kernel"] for c in multi} == {"mfma"}  # only the MFMA kernel takes several tokens
    assert at.build_config_space("prefill") == [{"kernel": "pingpong"}, {"kernel": "wide"}, {"kernel": "4wave"},
                                                {"kernel": "4wave_split"}]
    assert at.build_config_space("prefill_paged") == [{"kernel": "pingpong"}, {"kernel": "4wave"},
                                                      {"kernel": "4wave_split"}]
    with pytest.raises(ValueError):
        at.build_config_space("train")


def test_autotune_ranks_and_saves(tmp_path):
    path = tmp_path / "store.json"
    cost = {"a": 3.0, "b": 1.0, "c": 2.0}
    clock = {"t": 0.0}

    def runner(cfg):
        if cfg["kernel"] == "bad":
            raise RuntimeError("rejected by the library")
        clock["t"] += cost[cfg["kernel"]]

    import time as _time

    real = _time.perf_counter_ns
    try:
        _time.perf_counter_ns = lambda: int(clock["t"] * 1e9)  # deterministic CPU timing
        with pytest.warns(RuntimeWarning, match="skipped"):
            rows = at.autotune({"kind": "prefill", "signature": "S", "runner": runner, "flops": 4e9, "bytes": 2e9,
                                "default": {"kernel": "a"}},
                               [{"kernel": k} for k in ("a", "b", "bad", "c")], warmup=1, iters=3, path=path)
    finally:
        _time.perf_counter_ns = real
    assert [r["kernel"] for r in rows] == ["b", "c", "a"] and [r["rank"] for r in rows] == [1, 2, 3]
    assert rows[0]["latency_ms"] == pytest.approx(1000.0) and rows[0]["gbytes_per_s"] == pytest.approx(2.0)
    assert at.best_config("prefill", "S", path=path) == {"kernel": "b"}
    import json

    metrics = json.loads(path.read_text())["configs"]["prefill:S"]["metrics"]
    assert metrics["default_ms"] == pytest.approx(3000.0) and metrics["latency_ms"] == pytest.approx(1000.0)
    with pytest.raises(ValueError, match="missing"):
        at.autotune({"kind": "prefill"}, [{"kernel": "a"}])


def test_decode_and_prefill_wrappers_consult_the_store(tmp_path, monkeypatch):
    """config=None resolves through the store (no device work: CPU tensors)."""
    import torch

    from flashattntile_amd.kernels import decode as dec
    from flashattntile_amd.kernels import prefill as pre
    from flashattntile_amd.paging import allocate

    cache = allocate(batch=2, max_seq_len=64, num_kv_heads=2, head_dim=64, page_size=16, dtype=torch.float16,
                     device="cpu")
    q = torch.zeros(2, 8, 64, dtype=torch.float16)
    path = tmp_path / "store.json"
    monkeypatch.setenv("FAT_TUNED_CONFIGS", str(path))
    heuristic = dec._resolve_config(None, q, cache, 64, 8)
    assert heuristic["kernel"] is None and heuristic["split_k"] >= 1
    sig = at.decode_signature(2, 8, 2, 64, 16, 64, 8, torch.float16)
    at.save_best("decode", sig, {"split_k": 2, "pages_per_split": 0, "num_warps": 8, "kernel": "mfma"})
    got = dec._resolve_config(None, q, cache, 64, 8)
    assert (got["split_k"], got["pages_per_split"], got["num_warps"], got["kernel"]) == (2, 0, 8, "mfma")
    # an explicit config never reads the store (decode.py:474-500)
    assert dec._resolve_config({"split_k": 1}, q, cache, 64, 8)["kernel"] is None
    # another length is another shape: heuristic
    assert dec._resolve_config(None, q, cache, 48, 6) == dec._resolve_config(None, q, cache, 48, 6)
    assert dec._resolve_config(None, q, cache, 48, 6)["kernel"] is None
    # an entry the checks reject is ignored with a warning
    at.save_best("decode", sig, {"split_k": 99})
    with pytest.warns(RuntimeWarning, match="ignoring the stored decode config"):
        assert dec._resolve_config(None, q, cache, 64, 8) == heuristic
    # a VALU entry under a multi-token signature cannot run: ignored
    sig4 = at.decode_signature(2, 8, 2, 64, 16, 64, 8, torch.float16, q_len=4)
    at.save_best("decode", sig4, {"split_k": 1, "kernel": "valu"})
    q4 = torch.zeros(2, 4, 8, 64, dtype=torch.float16)
    with pytest.warns(RuntimeWarning, match="one query per sequence"):
        assert dec._resolve_config(None, q4, cache, 64, 8, q_len=4)["kernel"] is None
    # prefill: the reference's signature, the gfx950 knob
    psig = at.prefill_signature(1, 32, 8, 128, 512, 512, True)
    assert pre._resolve_config(None, "prefill", psig)["kernel"] is None
    at.save_best("prefill", psig, {"kernel": "4wave", "BLOCK_M": 128})
    cfg = pre._resolve_config(None, "prefill", psig)
    assert cfg["kernel"] == "4wave" and cfg["BLOCK_M"] == pre.DEFAULT_CONFIG["BLOCK_M"]
    assert pre._resolve_config({"kernel": "pingpong"}, "prefill", psig)["kernel"] == "pingpong"
    with pytest.raises(ValueError, match="kernel"):
        pre._resolve_config({"kernel": "8wave"})
    with pytest.raises(ValueError, match="unknown prefill config keys"):
        pre._resolve_config({"BLOCK_K": 64})
