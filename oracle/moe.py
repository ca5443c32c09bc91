"""MoE expert forwards on the CPU (oracle, test infrastructure only).

Three restatements, all over the SAME dequantized weights:

``forward_fp32``        the fidelity anchor of ``tests/test_fast.py:49-68`` (fp32 forward over
                        the dequantized NF4 values, ``index_add_`` of ``h * w``), accumulated
                        here in fp64 and returned as fp32.
``forward_fused_numerics``  the rounding points of the fused path ``engines/fast.py:100-160``:
                        bf16 gate_up output, the base epilogue in bf16 (``lora.py:102-128``), bf16
                        down output, fp32 router weight, ``buf[order] = down * w`` then a
                        fixed-axis k-sum (``fast.py:260-278``), cast back.
``forward_lora_fp32``   the same fp32 oracle for an ``ExpertsLoRA`` (``lora.py:329-407``): each
                        projection plus its low-rank delta ``scaling * (x A^T) B^T``
                        (``_lora``, ``lora.py:251-256``) before the activation, exact (fp64).
``reference_lora_loop`` ``ExpertsLoRA.forward`` itself in torch on the CPU, with its rounding
                        points (compute-dtype projections, the delta in the adapter dtype then
                        cast back, ``lora.py:251-256, 329-460``): the LoRA error anchor.
``reference_loop``      the reference per-expert loop ``ExpertsNbit.forward``
                        (``_vendor/experts.py:468-516``) in torch on the CPU: per hit expert,
                        dequantize to the compute dtype, ``F.linear``, ``act(gate) * up``,
                        ``F.linear``, a compute-dtype router-weight multiply (``:512``), fp32
                        ``index_add_`` (``:513``). This is the timed CPU baseline.

Epilogues (``epilogue`` argument): ``"swiglu"`` (``lora.py:125-127``), ``"act"`` (has_gate=False,
``lora.py:128``), ``("clamp_swiglu", limit)`` (DeepSeek-V4 ``_apply_gate``,
``arch/deepseek_v4.py:178-195``: fp32 GLU then cast), ``("gptoss", alpha, limit)`` with biases
(``arch/gptoss.py:100-112``; grouped form ``engines/hot_residency.py:72-80``).
"""
from __future__ import annotations

import numpy as np

from .numerics import round_to, sigmoid_f32, silu_f32
from .routing import route


def _epi_kind(epilogue):
    if isinstance(epilogue, tuple):
        return epilogue[0], epilogue[1:]
    return epilogue, ()


def _glu_exact(proj, epilogue, n_half):
    """fp64 epilogue on fp64 projections (no rounding): the oracle's activation."""
    kind, params = _epi_kind(epilogue)
    silu = lambda v: v / (1.0 + np.exp(-v))  # noqa: E731
    if kind == "act":
        return silu(proj)
    g, u = proj[:, :n_half], proj[:, n_half:]
    if kind == "swiglu":
        return silu(g) * u
    if kind == "clamp_swiglu":
        (limit,) = params
        if limit > 0:
            g = np.minimum(g, limit)
            u = np.clip(u, -limit, limit)
        return silu(g) * u
    if kind == "gptoss":
        alpha, limit = params
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
        return (u + 1.0) * (g * (1.0 / (1.0 + np.exp(-g * alpha))))
    raise ValueError(f"unknown epilogue {epilogue!r}")


def forward_fp32(x, top_k_index, top_k_weights, w1, w2, epilogue="swiglu", b1=None, b2=None):
    """fp32 oracle forward (``tests/test_fast.py:49-68``), accumulated in fp64.

    ``w1 [E, N1, K1]``, ``w2 [E, N2, K2]`` are the dequantized weights (fp32 values), ``x [T, H]``.
    Biases (gpt-oss) are added to the projections before the activation / after the down.
    """
    x = np.asarray(x, dtype=np.float64)
    idx = np.asarray(top_k_index, dtype=np.int64)
    wts = np.asarray(top_k_weights, dtype=np.float64)
    E = w1.shape[0]
    n_half = w1.shape[1] // 2
    out = np.zeros((x.shape[0], w2.shape[1]), dtype=np.float64)
    for e in range(E):
        tok, pos = np.nonzero(idx == e)
        if tok.size == 0:
            continue
        p = x[tok] @ np.asarray(w1[e], dtype=np.float64).T
        if b1 is not None:
            p = p + np.asarray(b1[e], dtype=np.float64)
        h = _glu_exact(p, epilogue, n_half)
        y = h @ np.asarray(w2[e], dtype=np.float64).T
        if b2 is not None:
            y = y + np.asarray(b2[e], dtype=np.float64)
        np.add.at(out, tok, y * wts[tok, pos][:, None])
    return out.astype(np.float32)


def forward_lora_fp32(x, top_k_index, top_k_weights, w1, w2, lora1, lora2, scaling, epilogue="swiglu"):
    """fp32 oracle of ``ExpertsLoRA.forward`` (``lora.py:329-407``), accumulated in fp64.

    ``lora1 = (A1 [E, r, K1], B1 [E, N1, r])`` and ``lora2 = (A2 [E, r, K2], B2 [E, N2, r])``.
    Per routed expert ``e`` with rows ``x_e``:
    ``proj = x_e W1[e]^T + scaling * (x_e A1[e]^T) B1[e]^T`` (``lora.py:373-382``: base
    projection plus ``_lora``), ``h = epilogue(proj)`` (``:384``, ``_epilogue`` at ``:102-128``),
    ``y = h W2[e]^T + scaling * (h A2[e]^T) B2[e]^T`` (``:386-399``), then ``y * w`` summed into the
    token (``:401-402``). No intermediate rounding. ``w1[e]`` / ``w2[e]`` may be any object
    indexable by expert (only the routed experts are read).
    """
    x = np.asarray(x, dtype=np.float64)
    idx = np.asarray(top_k_index, dtype=np.int64)
    wts = np.asarray(top_k_weights, dtype=np.float64)
    A1, B1 = (np.asarray(t, np.float64) for t in lora1)
    A2, B2 = (np.asarray(t, np.float64) for t in lora2)
    n_half = B1.shape[1] // 2
    out = np.zeros((x.shape[0], B2.shape[1]), dtype=np.float64)
    for e in sorted(set(idx.reshape(-1).tolist())):
        tok, pos = np.nonzero(idx == e)
        xe = x[tok]
        p = xe @ np.asarray(w1[e], np.float64).T + scaling * ((xe @ A1[e].T) @ B1[e].T)
        h = _glu_exact(p, epilogue, n_half)
        y = h @ np.asarray(w2[e], np.float64).T + scaling * ((h @ A2[e].T) @ B2[e].T)
        np.add.at(out, tok, y * wts[tok, pos][:, None])
    return out.astype(np.float32)


def reference_lora_loop(x, top_k_index, top_k_weights, w1_dq, w2_dq, lora1, lora2, scaling, num_experts,
                        compute_dtype=None, has_gate=True):
    """``ExpertsLoRA.forward`` (``lora.py:329-407``; one token: ``_forward_decode``, ``:409-460``) in
    torch on the CPU with the reference's rounding points: base projections in the compute dtype
    (``F.linear`` against the dequantized expert), ``_lora`` in the adapter dtype and cast back
    (``:251-256``), the SwiGLU in the compute dtype, the router weight multiplied in the compute
    dtype and accumulated in fp32. ``w1_dq`` / ``w2_dq`` are ``(e, dtype) -> [out, in]`` callables;
    ``lora1`` / ``lora2`` are ``(A, B)`` torch tensors. Returns ``x``'s dtype."""
    import torch
    import torch.nn.functional as F

    def _lora(v, A, B):
        return (scaling * F.linear(F.linear(v.to(A.dtype), A), B)).to(v.dtype)

    def _act(proj):
        if has_gate:
            g, u = proj.chunk(2, dim=-1)
            return F.silu(g) * u
        return F.silu(proj)

    input_dtype = x.dtype
    cd = compute_dtype if compute_dtype is not None else x.dtype
    hs = x.to(cd)
    A1, B1 = lora1
    A2, B2 = lora2
    final = torch.zeros_like(hs, dtype=torch.float32)
    with torch.no_grad():
        if hs.shape[0] == 1:  # _forward_decode: the token's slots in routing order
            for j in range(top_k_index.shape[1]):
                e = int(top_k_index[0, j])
                proj = F.linear(hs, w1_dq(e, cd)) + _lora(hs, A1[e], B1[e])
                h = _act(proj)
                h = F.linear(h, w2_dq(e, cd)) + _lora(h, A2[e], B2[e])
                final += (h * top_k_weights[0, j]).to(final.dtype)
            return final.to(input_dtype)
        mask = F.one_hot(top_k_index, num_classes=num_experts).permute(2, 1, 0)
        hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero(as_tuple=False).view(-1)
        for e in hit.tolist():
            pos, tok = torch.where(mask[e])
            cur = hs[tok]
            proj = F.linear(cur, w1_dq(e, cd)) + _lora(cur, A1[e], B1[e])
            h = _act(proj)
            h = F.linear(h, w2_dq(e, cd)) + _lora(h, A2[e], B2[e])
            h = h * top_k_weights[tok, pos, None]
            final.index_add_(0, tok, h.to(final.dtype))
    return final.to(input_dtype)


def epilogue_rounded(proj_r, epilogue, n_half, dt="bf16", b1=None):
    """The fused path's epilogue with the reference's rounding points (inputs already rounded
    to ``dt``). Restates ``lora.py:125-128`` (torch ops on ``dt`` tensors round after every op),
    ``deepseek_v4.py:190-195`` (fp32 GLU, one rounding), ``hot_residency.py:72-80`` (gpt-oss)."""
    kind, params = _epi_kind(epilogue)
    r = lambda v: round_to(np.asarray(v, np.float32), dt)  # noqa: E731
    p = np.asarray(proj_r, np.float32)
    if kind == "gptoss":
        p = r(p + np.asarray(b1, np.float32))
    if kind == "act":
        return r(silu_f32(p))
    g, u = p[:, :n_half], p[:, n_half:]
    if kind == "swiglu":
        return r(r(silu_f32(g)) * u)
    if kind == "clamp_swiglu":
        (limit,) = params
        if limit > 0:
            g = np.minimum(g, np.float32(limit))
            u = np.clip(u, np.float32(-limit), np.float32(limit))
        return r(silu_f32(g) * u)
    if kind == "gptoss":
        alpha, limit = params
        g = np.minimum(g, np.float32(limit))
        u = np.clip(u, np.float32(-limit), np.float32(limit))
        t = r(g * np.float32(alpha))
        sg = r(sigmoid_f32(t))
        gs = r(g * sg)
        u1 = r(u + np.float32(1.0))
        return r(u1 * gs)
    raise ValueError(f"unknown epilogue {epilogue!r}")


def forward_fused_numerics(x, top_k_index, top_k_weights, w1, w2, epilogue="swiglu", dt="bf16",
                           b1=None, b2=None, out_dtype="bf16"):
    """The fused path's rounding points (``engines/fast.py:100-160, 260-278``), fp32 GEMMs.

    Rows are processed in the sorted (expert-grouped) order of ``route``; every group's GEMM
    accumulates in fp32 (numpy sgemm) and rounds to ``dt``; the combine multiplies the
    ``dt``-rounded down output by the fp32 router weight and sums the k slots in slot order.
    """
    x = np.asarray(x, np.float32)
    idx = np.asarray(top_k_index, np.int64)
    T, k = idx.shape
    E = w1.shape[0]
    n_half = w1.shape[1] // 2
    rt = route(idx, E)
    a = round_to(x[rt["token_rows"]], dt)
    M = a.shape[0]
    H2 = w2.shape[1]
    down = np.zeros((M, H2), np.float32)
    for e in rt["active"]:
        s, t = rt["offsets"][e], rt["offsets"][e + 1]
        up = round_to(a[s:t] @ np.asarray(w1[e], np.float32).T, dt)
        bias1 = None if b1 is None else round_to(np.asarray(b1[e], np.float32), dt)
        h = epilogue_rounded(up, epilogue, n_half, dt, bias1)
        dn = round_to(h @ np.asarray(w2[e], np.float32).T, dt)
        if b2 is not None:
            dn = round_to(dn + round_to(np.asarray(b2[e], np.float32), dt), dt)
        down[s:t] = dn
    w = np.asarray(top_k_weights, np.float32)[rt["token_rows"], rt["top_pos"]]
    buf = np.zeros((T * k, H2), np.float32)
    buf[rt["order"]] = down * w[:, None]
    acc = np.zeros((T, H2), np.float32)
    b3 = buf.reshape(T, k, H2)
    for s in range(k):
        acc = (acc + b3[:, s, :]).astype(np.float32)
    return round_to(acc, out_dtype)


def reference_loop(x, top_k_index, top_k_weights, w1_dq, w2_dq, num_experts, compute_dtype=None,
                   has_gate=True):
    """Reference per-expert loop ``ExpertsNbit.forward`` (``_vendor/experts.py:468-516``), torch CPU.

    ``w1_dq`` / ``w2_dq`` are callables ``(e, dtype) -> torch.Tensor [out, in]`` returning the
    dequantized expert (the reference's ``_dequantize_expert``), so the dequant cost sits inside
    the loop exactly where the reference pays it. Returns a torch tensor in ``x``'s dtype.
    """
    import torch
    import torch.nn.functional as F

    input_dtype = x.dtype
    cd = compute_dtype if compute_dtype is not None else x.dtype
    hs = x.to(cd)
    final = torch.zeros_like(hs, dtype=torch.float32)
    with torch.no_grad():
        mask = F.one_hot(top_k_index, num_classes=num_experts).permute(2, 1, 0)
        hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero(as_tuple=False).view(-1)
        for e in hit.tolist():
            pos, tok = torch.where(mask[e])
            cur = hs[tok]
            proj = F.linear(cur, w1_dq(e, cd))
            if has_gate:
                g, u = proj.chunk(2, dim=-1)
                h = F.silu(g) * u
            else:
                h = F.silu(proj)
            h = F.linear(h, w2_dq(e, cd))
            h = h * top_k_weights[tok, pos, None]
            final.index_add_(0, tok, h.to(final.dtype))
    return final.to(input_dtype)


def dequant_torch_expert(packed_e, absmax_e, code, n, k, dtype):
    """``cold_engine.py:104-115`` ``_dequant_torch`` for one expert, then the cast to ``dtype``."""
    import torch

    pk = packed_e.reshape(-1)
    idx = torch.empty(pk.numel() * 2, dtype=torch.long)
    idx[0::2] = (pk >> 4).long()
    idx[1::2] = (pk & 0xF).long()
    vals = code.index_select(0, idx)
    return (vals.reshape(-1, 64) * absmax_e.reshape(-1, 1)).reshape(n, k).to(dtype)


def rel_errors(got, want):
    """(rel-Frobenius, max-abs on unit-scale outputs, max-abs / max|want|) of ``[tokens, hidden]``
    outputs. "Unit-scale" puts every token's output row at unit RMS (the oracle row's RMS), so a
    token whose routing weights make its output several times larger than another's is not
    judged on that scale; ``max-abs / max|want|`` is the reference's own ``_b_rel``
    (``tests/test_fast.py:43-46``)."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    if not w.size:
        return 0.0, 0.0, 0.0
    fro = np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30)
    w2 = w.reshape(-1, w.shape[-1])
    rms = np.maximum(np.sqrt(np.mean(w2 * w2, axis=-1, keepdims=True)), 1e-30)
    maxabs = np.max(np.abs(g.reshape(w2.shape) - w2) / rms)
    brel = np.max(np.abs(g - w)) / max(np.max(np.abs(w)), 1e-30)
    return float(fro), float(maxabs), float(brel)


def maxabs_global_rms(got, want):
    """max-abs over the whole output divided by the whole output's RMS (one scale for all
    tokens): a stricter figure than ``rel_errors``' per-token one, reported beside it."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    rms = max(np.sqrt(np.mean(w * w)) if w.size else 0.0, 1e-30)
    return float(np.max(np.abs(g - w)) / rms) if w.size else 0.0
