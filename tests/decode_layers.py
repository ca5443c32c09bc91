"""Single-token MoE layers for the decode-path GPU tests: quantized weight stacks built from a
seed, their oracle decode (the C restatement, never the kernels under test), seeded inputs and
the layer bars (rel-Frobenius <= 1e-2, max-abs <= 2e-2 of the oracle row RMS)."""
import numpy as np
import torch

from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import ops, quant as Q
from oracle import c_oracle, moe

DEV = "cuda"


def _dense(qw) -> np.ndarray:
    """``[E, n, k]`` fp32 weights of a descriptor decoded by the oracle's C restatement."""
    E, n, k = qw.num_experts, qw.n, qw.k
    packed = qw.packed.cpu().numpy().reshape(E, -1)
    absmax = qw.absmax.cpu().numpy().reshape(E, -1)
    out = np.empty((E, n, k), np.float32)
    for e in range(E):
        if qw.fmt == N.FMT_MXFP4:
            out[e] = c_oracle.dequant_mxfp4(packed[e], absmax[e], n, k)
            continue
        am = absmax[e]
        if qw.fmt == N.FMT_NF4_DQ:
            am = c_oracle.dequant_absmax_dq(am, qw.absmax2.cpu().numpy().reshape(E, -1)[e],
                                            float(qw.offset.cpu().numpy().reshape(E)[e]), qw.code2.cpu().numpy())
        out[e] = c_oracle.dequant_4bit(packed[e], am, qw.code.cpu().numpy()).reshape(n, k)
    return out


def _stack(fmt, E, n, k, seed, code=None):
    g = torch.Generator().manual_seed(seed)
    if fmt == "mxfp4":
        w = torch.randn(E, n, k, generator=g) * 0.05
        b, s = Q.quantize_mxfp4(w)
        return ops.mxfp4_qweight(b.reshape(E, -1).to(DEV), s.reshape(E, -1).to(DEV), n, k, num_experts=E)
    w = torch.randn(E, n * k, generator=g) * 0.02
    packed, absmax = Q.quantize_4bit(w)
    code = code if code is not None else Q.code_4bit("nf4").to(DEV)
    if fmt == "nf4_dq":
        q, a2, off = Q.double_quant(absmax)
        return ops.nf4_dq_qweight(packed.to(DEV), q.to(DEV), a2.to(DEV), off.to(DEV), code,
                                  Q.dynamic_map().to(DEV), n, k, num_experts=E)
    return ops.nf4_qweight(packed.to(DEV), absmax.to(DEV), code, n, k, num_experts=E)


class Layer:
    """One MoE layer's quantized weights (and their oracle decode, made on first use)."""

    def __init__(self, fmt, E, H, I, dt, seed=60):
        self.fmt, self.E, self.H, self.I, self.dt = fmt, E, H, I, dt
        # one code table for both projections, as a module has
        code = Q.code_4bit("nf4").to(DEV)
        self.w1 = _stack(fmt, E, 2 * I, H, seed, code)
        self.w2 = _stack(fmt, E, H, I, seed + 1, code)
        self.epi, self.spec, self.limit = N.EPI_SWIGLU, "swiglu", 7.0
        if fmt == "mxfp4":  # gpt-oss: biases in the activation type, clamped GLU
            g = torch.Generator().manual_seed(seed + 2)
            self.w1.bias = (torch.randn(E, 2 * I, generator=g) * 0.1).to(dt).to(DEV)
            self.w2.bias = (torch.randn(E, H, generator=g) * 0.1).to(dt).to(DEV)
            self.epi, self.spec = N.EPI_GPTOSS, ("gptoss", 1.702, 7.0)
        self._dense = None

    def dense(self):
        if self._dense is None:
            self._dense = (_dense(self.w1), _dense(self.w2))
        return self._dense

    def run(self, x, idx, wts, path=N.PATH_AUTO, out_dtype=torch.float32):
        return ops.moe_forward(x, idx, wts, self.w1, self.w2, self.epi, out_dtype, limit=self.limit, path=path)

    def oracle(self, x, idx, wts):
        W1, W2 = self.dense()
        b1 = None if self.w1.bias is None else self.w1.bias.float().cpu().numpy()
        b2 = None if self.w2.bias is None else self.w2.bias.float().cpu().numpy()
        return moe.forward_fp32(x.float().cpu().numpy(), idx.cpu().numpy(), wts.float().cpu().numpy(), W1, W2,
                                self.spec, b1, b2)


def _inputs(E, H, top, seed, dt, ids=None):
    rng = np.random.default_rng(seed)
    idx = np.asarray(ids if ids is not None else rng.permutation(E)[:top][None, :], np.int64)
    x = (torch.randn(1, H, generator=torch.Generator().manual_seed(seed)) * 2).to(dt)
    wts = torch.rand(1, idx.shape[1], generator=torch.Generator().manual_seed(seed + 1)).to(torch.bfloat16)
    return x.to(DEV), torch.from_numpy(idx).to(DEV), wts.to(DEV)


def _check(got, want, what):
    fro, maxabs, _ = moe.rel_errors(got.float().cpu().numpy(), want)
    assert fro <= 1e-2 and maxabs <= 2e-2, (what, fro, maxabs)
    return fro, maxabs


