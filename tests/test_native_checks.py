"""The native decode entry's argument checks, on the CPU.

``native.paged_decode_attention`` makes the reference binding's checks
(csrc/paged_decode.cu:306-323, ``TORCH_CHECK`` -> ``RuntimeError``) before
anything is enqueued.  They read only tensor metadata, so they are exercised
here on CPU tensors wrapped to report a ROCm device; nothing launches."""

from __future__ import annotations

import pytest
import torch

from flashattntile_amd import native


class OnDevice:
    """A CPU tensor's metadata, reported as living on ROCm device 0."""

    is_cuda = True

    def __init__(self, t: torch.Tensor, on_device: bool = True) -> None:
        self.t = t
        self.is_cuda = on_device

    def dim(self):
        return self.t.dim()

    def is_contiguous(self):
        return self.t.is_contiguous()

    @property
    def dtype(self):
        return self.t.dtype

    @property
    def shape(self):
        return self.t.shape

    @property
    def device(self):
        return torch.device("cuda", 0) if self.is_cuda else self.t.device


def _args(**over):
    q = torch.zeros(2, 8, 128, dtype=torch.float16)
    k = torch.zeros(6, 16, 2, 128, dtype=torch.float16)
    base = {"q": q, "k": k, "v": k.clone(), "pt": torch.zeros(2, 3, dtype=torch.int32),
            "sl": torch.ones(2, dtype=torch.int32), "P": 16}
    base.update(over)
    wrap = {n: OnDevice(t) if isinstance(t, torch.Tensor) else t for n, t in base.items()}
    return wrap["q"], wrap["k"], wrap["v"], wrap["pt"], wrap["sl"], wrap["P"]


CASES = [
    ({"q": OnDevice(torch.zeros(2, 8, 128, dtype=torch.float16), on_device=False)}, "q must be a CUDA tensor"),
    ({"v": OnDevice(torch.zeros(6, 16, 2, 128, dtype=torch.float16), on_device=False)},
     "KV cache must be CUDA tensors"),
    ({"sl": OnDevice(torch.ones(2, dtype=torch.int32), on_device=False)}, "metadata must be CUDA tensors"),
    ({"q": torch.zeros(8, 128, dtype=torch.float16)}, r"q must be \[batch, heads, head_dim\]"),
    ({"k": torch.zeros(6, 16, 256, dtype=torch.float16)}, r"cache must be \[pages, page, kv, dim\]"),
    ({"q": torch.zeros(8, 2, 128, dtype=torch.float16).transpose(0, 1)}, "q must be contiguous"),
    ({"k": torch.zeros(6, 2, 16, 128, dtype=torch.float16).transpose(1, 2)}, "cache must be contiguous"),
    ({"pt": torch.zeros(2, 3, dtype=torch.int64)}, "page_table must be int32"),
    ({"sl": torch.ones(2, dtype=torch.int64)}, "seq_lens must be int32"),
    ({"q": torch.zeros(2, 8, 128, dtype=torch.bfloat16)}, "q and cache dtypes must match"),
    ({"v": torch.zeros(7, 16, 2, 128, dtype=torch.float16)}, "k/v cache shapes must match"),
    ({"q": torch.zeros(2, 8, 64, dtype=torch.float16)}, "q head_dim must match cache head_dim"),
    ({"P": 0}, r"page_size must be in \[1, 32\]"),
    ({"P": 64}, r"page_size must be in \[1, 32\]"),
    ({"pt": torch.zeros(3, 3, dtype=torch.int32)}, "page_table batch must match q"),
    ({"sl": torch.ones(1, dtype=torch.int32)}, "seq_lens batch must match q"),
    ({"q": torch.zeros(2, 7, 128, dtype=torch.float16)}, "heads must be divisible by KV heads"),
    ({"P": 32}, "exceeds the cache's page dimension"),
]


@pytest.mark.parametrize("over,msg", CASES, ids=[m for _, m in CASES])
def test_binding_checks(over, msg):
    with pytest.raises(RuntimeError, match=msg):
        native._check_args(*_args(**over))


def test_dtype_and_head_dim_limits():
    q = torch.zeros(2, 8, 96, dtype=torch.float16)
    k = torch.zeros(6, 16, 2, 96, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="head_dim 64 or 128"):
        native._check_args(*_args(q=q, k=k, v=k.clone()))
    q8 = torch.zeros(2, 8, 128, dtype=torch.int8)
    k8 = torch.zeros(6, 16, 2, 128, dtype=torch.int8)
    with pytest.raises(RuntimeError, match="fp16, bf16 and fp32"):
        native._check_args(*_args(q=q8, k=k8, v=k8.clone()))
    for dt in (torch.float16, torch.bfloat16, torch.float32):  # accepted, with page sizes 1..16 here
        for P in (1, 3, 16):
            q = torch.zeros(2, 8, 64, dtype=dt)
            k = torch.zeros(6, 16, 2, 64, dtype=dt)
            native._check_args(*_args(q=q, k=k, v=k.clone(), P=P))


def test_unavailable_path_raises_without_a_device():
    if native.is_available():
        pytest.skip("a ROCm device is present")
    assert native.unavailable_reason()
    q = torch.zeros(1, 2, 64, dtype=torch.float16)
    k = torch.zeros(1, 16, 1, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="native HIP path unavailable"):
        native.paged_decode_attention(q, k, k, torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32),
                                      16)
