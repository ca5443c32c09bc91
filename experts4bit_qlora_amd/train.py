"""The training lane: ``enable_fast_train`` routes an ``ExpertsLoRA``'s training forward AND
backward through the gfx950 kernels (reference ``experts4bit_qlora/engines/fast.py:453-674``).

Forward, per projection (``_GroupedLoraProj``), over expert-sorted rows and with no host sync
(the reference sorts with ``argsort`` and reads group sizes back with ``.tolist()``):

    proj[m] = a_m . deq(W[e_m])^T + scaling * (a_m . A[e_m]^T) . B[e_m]^T

one grouped GEMM to fp32 rows, ``t = a . A^T`` kept for the backward, the delta added in fp32,
one rounding to the compute dtype. The base's own ``_epilogue`` sits between the two projections
(``act(Wx + BAx)``, so the delta must land before it), and the router weights combine the down
rows in fp32 (``fast.py:260-278``'s ``_scatter_combine``), both as differentiable torch ops.

Backward of a projection, from ``g = dL/dproj`` (compute dtype, sorted rows):

    dL/da_m  = g_m . deq(W[e_m]) + scaling * (g_m . B[e_m]) . A[e_m]     e4b_grouped_dgrad,
                                                                            e4b_lora_t, e4b_lora_t_add
    dL/dA[e] = scaling * sum_{m in e} (g_m . B[e])^T a_m                   e4b_lora_wgrad
    dL/dB[e] = scaling * sum_{m in e} g_m^T t_m                            e4b_lora_wgrad

and, for the gate_up projection, whose rows gather the tokens, ``dL/dx[t]`` sums its k rows in
slot order. The frozen weights are decoded inside the dgrad kernel (never materialised), as the
reference's ``nf4_qlora.fused_grouped_lora`` recompute-decode backward does.

``dgrad`` (``enable_fast_train(..., dgrad=True)``) is accepted and recorded like the reference's
flag, but both settings run the same single-launch HIP dgrad: there is no per-expert decode
loop to fall back to here.
"""
from __future__ import annotations

import types
import warnings

import torch

from . import _native as N
from . import ops


class _GroupedLoraProj(torch.autograd.Function):
    """``proj = a . deq(W)^T + scaling * (a . A^T) . B^T`` over expert-sorted rows; see the module
    docstring for the backward."""

    @staticmethod
    def forward(ctx, a, lora_a, lora_b, qw, rb, M, E, gather_k, tokens, scaling, out_dtype):
        proj = ops.grouped_gemm(a, qw, rb, tokens, M, N.EPI_NONE, gather_k=gather_k, path=N.PATH_MFMA,
                                out_dtype=torch.float32)
        t = ops.lora_t(a, rb, M, E, lora_a, gather_k=gather_k)
        ops.lora_t_add(t, rb, M, E, lora_b, scaling, proj, delta_dtype=torch.float32)
        ctx.save_for_backward(a, lora_a, lora_b, t)
        ctx.qw, ctx.rb, ctx.M, ctx.E, ctx.gather_k, ctx.scaling = qw, rb, M, E, gather_k, scaling
        return proj.to(out_dtype)

    @staticmethod
    def backward(ctx, g):
        a, lora_a, lora_b, t = ctx.saved_tensors
        qw, rb, M, E, gk, s = ctx.qw, ctx.rb, ctx.M, ctx.E, ctx.gather_k, ctx.scaling
        g = g.to(a.dtype).contiguous()
        need_a, need_A, need_B = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        grad_a = grad_A = grad_B = None
        u = None
        if need_a or need_A:
            # u[m] = g_m . B[e_m]: the t pass over B^T ([E, r, n])
            u = ops.lora_t(g, rb, M, E, lora_b.transpose(1, 2).contiguous())
        if need_a:
            da = ops.grouped_dgrad(g, qw, rb, M)  # fp32 [M, k]
            # + scaling * u . A[e]: the delta pass with A^T ([E, k, r]) as its B
            ops.lora_t_add(u, rb, M, E, lora_a.transpose(1, 2).contiguous(), s, da, delta_dtype=torch.float32)
            if gk > 0:
                # token t's gradient: its k sorted rows, summed in slot order
                inv = rb.inv[:M].long()
                T = M // gk
                grad_a = da.index_select(0, inv.clamp_min(0)).mul_((inv >= 0).unsqueeze(1)).view(T, gk, -1).sum(1)
                grad_a = grad_a.to(a.dtype)
            else:
                grad_a = da.to(a.dtype)
        if need_A:
            grad_A = ops.lora_wgrad(u, a, rb, M, E, s, gather_k=gk).to(lora_a.dtype)
        if need_B:
            grad_B = ops.lora_wgrad(t, g, rb, M, E, s).transpose(1, 2).contiguous().to(lora_b.dtype)
        return grad_a, grad_A, grad_B, None, None, None, None, None, None, None, None


def _train_tile_m(M: int, E: int) -> int:
    """Row tiles of the training GEMMs: 128 once experts average 64 rows or more, else 32 (the
    forward's rule)."""
    return ops.mfma_tile_m() if M >= 64 * min(E, M) else 32


def fused_experts_train_forward(lora_mod, hidden_states, top_k_index, top_k_weights):
    """Training-capable fused forward of an ``ExpertsLoRA`` (``fast.py:453-556``): both projections
    through ``_GroupedLoraProj``, the base's own epilogue between them, the fp32 router-weighted
    combine, all differentiable; evicted storage or a non-bf16/fp16 compute dtype runs the saved
    reference forward."""
    from . import fast as F
    from .lora import _epilogue

    base = lora_mod.base
    input_dtype = hidden_states.dtype
    compute_dtype = base.compute_dtype if base.compute_dtype is not None else input_dtype
    if compute_dtype not in (torch.bfloat16, torch.float16) or base.gate_up_proj.numel() == 0 \
            or base.down_proj.numel() == 0:
        return lora_mod._e4b_train_ref(hidden_states, top_k_index, top_k_weights)
    x = hidden_states.to(compute_dtype)
    tokens = x.shape[0]
    k = top_k_index.shape[1]
    hidden = base._down_shape[0]
    if tokens == 0:
        return x.new_zeros(0, hidden).to(input_dtype)
    E = base.num_experts
    M = tokens * k
    w1, w2 = F._qweights(base)
    rb = ops.route(top_k_index, E, tile_m=_train_tile_m(M, E))
    s = float(lora_mod.scaling)
    proj = _GroupedLoraProj.apply(x, lora_mod.gate_up_lora_A, lora_mod.gate_up_lora_B, w1, rb, M, E, k, tokens, s,
                                  compute_dtype)
    # the base's OWN epilogue (fast.py:525-528): clamps and custom activations included
    h = _epilogue(base, proj).to(compute_dtype).contiguous()
    down = _GroupedLoraProj.apply(h, lora_mod.down_lora_A, lora_mod.down_lora_B, w2, rb, M, E, 0, tokens, s,
                                  compute_dtype)
    # combine: out[t] = sum_s w[t, s] * down[row of (t, s)] in fp32, slots in order
    inv = rb.inv[:M].long()
    rows = down.index_select(0, inv.clamp_min(0)).float() * (inv >= 0).unsqueeze(1)
    w = top_k_weights.reshape(-1, 1).to(torch.float32)
    return (rows * w).view(tokens, k, hidden).sum(1).to(input_dtype)


def _train_eligible(mod):
    """None if ``mod`` (an ExpertsLoRA) can take the fused training lane, else why not."""
    from . import fast as F
    from .experts import Experts4bit, ExpertsNbit

    base = mod.base
    if type(base).forward not in {ExpertsNbit.forward, Experts4bit.forward} and not hasattr(base, "_apply_gate"):
        return f"base {type(base).__name__} has a custom forward"
    if getattr(base, "_e4b_mxfp4_arena", False):
        return "base storage is MXFP4 (arena); the NF4 grouped kernels cannot read it"
    why = F._eligible(base)
    if why is not None:
        return why
    n1, _ = base._gate_up_shape
    n2, _ = base._down_shape
    if n1 % 64 or n2 % 64:
        return "projection output features not divisible by 64 (the grouped dgrad's reduction step)"
    if mod.gate_up_lora_A.shape[1] > 64:
        return f"LoRA rank {mod.gate_up_lora_A.shape[1]} > 64"
    return None


def enable_fast_train(model, verbose: bool = False, dgrad: bool = False) -> int:
    """Route ``ExpertsLoRA`` TRAINING (forward and backward) through the HIP kernels; returns the
    number patched (``fast.py:557-658``). Idempotent: an already patched module is kept, with a
    warning when ``dgrad`` differs from its recorded flag; modules patched by a batched lane
    (``_e4b_batched_ref``), bases with a custom forward and MXFP4-arena bases are skipped. Returns
    0 when the kernel library is unavailable."""
    from .lora import ExpertsLoRA

    if not N.available():
        if verbose:
            print("[e4b.fast] the MI355X kernel library is unavailable: no fused training path")
        return 0
    mods = list(model.modules()) if hasattr(model, "modules") else [model]
    patched = 0
    for mod in mods:
        if not isinstance(mod, ExpertsLoRA):
            continue
        if hasattr(mod, "_e4b_train_ref"):
            if getattr(mod, "_e4b_dgrad", False) != dgrad:
                warnings.warn(
                    f"[e4b.fast] enable_fast_train(dgrad={dgrad}) on a module already patched with "
                    f"dgrad={getattr(mod, '_e4b_dgrad', False)}: the existing patch is kept and the flag is NOT "
                    "applied. Call disable_fast_train first to change it.", RuntimeWarning, stacklevel=2)
            continue
        if hasattr(mod, "_e4b_batched_ref"):
            if verbose:
                print("[e4b.fast] skip: enable_batched_train already patched this module; call "
                      "disable_batched_train first")
            continue
        why = _train_eligible(mod)
        if why is not None:
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: {why}")
            continue
        mod._e4b_train_ref = mod.forward
        mod._e4b_dgrad = dgrad
        mod.forward = types.MethodType(lambda self, hs, tki, tkw: fused_experts_train_forward(self, hs, tki, tkw),
                                       mod)
        patched += 1
    if verbose:
        print(f"[e4b.fast] fused TRAINING path on {patched} ExpertsLoRA module(s)")
    return patched


def disable_fast_train(model) -> int:
    """Restore the forwards ``enable_fast_train`` replaced (``fast.py:661-674``); returns the count."""
    n = 0
    mods = list(model.modules()) if hasattr(model, "modules") else [model]
    for mod in mods:
        ref = getattr(mod, "_e4b_train_ref", None)
        if ref is not None:
            mod.forward = ref
            del mod._e4b_train_ref
            if hasattr(mod, "_e4b_dgrad"):
                del mod._e4b_dgrad
            n += 1
    return n
