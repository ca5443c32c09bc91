"""e4b_moe_forward_noalloc: the forward with its workspace in the library's static device array.

Called through the C-ABI and checked against e4b_moe_forward (which takes a caller-allocated
workspace) on the same inputs: both run the same kernels, so the outputs must be bit-identical.
Two calls in a row, the second with a smaller input (the array keeps the first call's
contents), over the MFMA / fp16 matrix-core path (hundreds of tokens), the decode path and the
gpt-oss MXFP4 path; a call whose workspace exceeds the array is rejected before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import ops, quant as Q

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _nf4(E, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    packed, absmax = Q.quantize_4bit(torch.randn(E, n * k, generator=g) * 0.02)
    qw = ops.nf4_qweight(packed.to(DEV), absmax.to(DEV), Q.code_4bit("nf4").to(DEV), n, k, num_experts=E)
    return ops.with_weight_shift(qw)


def _mxfp4(E, n, k, seed, dt):
    g = torch.Generator().manual_seed(seed)
    b, s = Q.quantize_mxfp4(torch.randn(E, n, k, generator=g) * 0.05)
    qw = ops.mxfp4_qweight(b.reshape(E, -1).to(DEV), s.reshape(E, -1).to(DEV), n, k, num_experts=E)
    qw.bias = (torch.randn(E, n, generator=g) * 0.1).to(dt).to(DEV)
    return qw


def _inputs(E, H, T, top, seed, dt):
    rng = np.random.default_rng(seed)
    idx = torch.from_numpy(np.stack([rng.permutation(E)[:top] for _ in range(T)]).astype(np.int64)).to(DEV)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(seed)).to(dt).to(DEV)
    w = torch.rand(T, top, generator=torch.Generator().manual_seed(seed + 1)).to(torch.bfloat16).to(DEV)
    return x, idx, w


def _noalloc(x, idx, w, w1, w2, epi, out_dtype, alpha=1.702, limit=7.0):
    """One e4b_moe_forward_noalloc call through the C-ABI; returns (status, out)."""
    L = N.lib()
    T, k = idx.shape
    out = torch.empty(T, w2.n, dtype=out_dtype, device=x.device)
    s1, s2 = w1.struct(), w2.struct()
    st = L.e4b_moe_forward_noalloc(x.data_ptr(), ops.dtype_code(x.dtype), T, idx.data_ptr(), w.data_ptr(),
                                   ops.dtype_code(w.dtype), k, ctypes.byref(s1), ctypes.byref(s2), epi, alpha, limit,
                                   N.PATH_AUTO, out.data_ptr(), ops.dtype_code(out_dtype), ops._stream(x.device))
    return st, out


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_noalloc_matches_the_workspace_entry_point(fmt):
    dt = torch.bfloat16
    if fmt == "nf4":
        E, H, I, top, epi = 16, 1024, 512, 8, N.EPI_SWIGLU
        w1, w2 = _nf4(E, 2 * I, H, 1), _nf4(E, H, I, 2)
        sizes = (300, 5)  # MFMA GEMMs in fp16 mode, then the decode path
    else:
        E, H, I, top, epi = 8, 2880, 512, 4, N.EPI_GPTOSS
        w1, w2 = _mxfp4(E, 2 * I, H, 3, dt), _mxfp4(E, H, I, 4, dt)
        sizes = (96, 1)
    for i, T in enumerate(sizes):
        _announce(f"noalloc fmt={fmt} call={i} tokens={T}")
        x, idx, w = _inputs(E, H, T, top, 10 + i, dt)
        st, got = _noalloc(x, idx, w, w1, w2, epi, torch.float32)
        assert st == N.E4B_OK, N.lib().e4b_last_error().decode()
        want = ops.moe_forward(x, idx, w, w1, w2, epi, torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (fmt, i, T, (got - want).abs().max().item())


def test_noalloc_rejects_a_workspace_beyond_its_array():
    _announce("noalloc oversize")
    E, H, I, top = 16, 1024, 512, 8
    w1, w2 = _nf4(E, 2 * I, H, 5), _nf4(E, H, I, 6)
    L = N.lib()
    T = 8192  # far beyond 64 MiB of workspace at these sizes
    assert L.e4b_moe_workspace_bytes(T, top, E, w1.n, w2.n, N.EPI_SWIGLU, N.BF16) > N.NOALLOC_WORKSPACE_BYTES
    x = torch.zeros(T, H, dtype=torch.bfloat16, device=DEV)
    idx = torch.zeros(T, top, dtype=torch.int64, device=DEV)
    w = torch.zeros(T, top, dtype=torch.bfloat16, device=DEV)
    st, _ = _noalloc(x, idx, w, w1, w2, N.EPI_SWIGLU, torch.bfloat16)
    assert st == -4, st  # E4B_ESPACE
    assert "holds" in L.e4b_last_error().decode()
