"""``enable_fast``: route frozen expert modules through the gfx950 kernels.

Same entry points, eligibility rules, markers, return counts and fallbacks as the reference
(``experts4bit_qlora/engines/fast.py:66-423``):

* ``fast_available()`` -- the HIP library loads and a device is up.
* ``enable_fast(model, verbose=False) -> int`` patches every eligible ``ExpertsLoRA`` wrapper
  (skipping its wrapped base) and every eligible bare ``ExpertsNbit``; it sets
  ``mod._e4b_fast_ref = mod.forward`` and binds the fused forward; idempotent; mutually
  exclusive with the other engines' markers; warns in training mode.
* ``disable_fast(model) -> int`` restores the saved forwards.

The fused forwards keep the reference's positional signature ``(mod, hidden_states,
top_k_index, top_k_weights)`` (the offload pre-hook reads ``args[1]``) and fall back to the saved
reference forward when grad is required, in training mode (wrapper), for a non-bf16/fp16
compute dtype, or for an evicted (0-element) store.

Beyond the reference: ``GptOssExpertsMxfp4`` modules (MXFP4 + biases + clamped GLU) are fused
too, and NF4 with double-quantized absmax is eligible. Where the reference issues ~15 torch
launches and a device->host sync per layer (``fast.py:125-160``), the bare fused forward here is
ONE library call (route, gate_up + epilogue, down, combine) with no host sync.
"""
from __future__ import annotations

import weakref
from typing import Optional

import torch
import torch.nn.functional as F

from . import _native as N
from . import ops
from .arch.deepseek_v4 import _DeepseekV4ForwardMixin
from .arch.gptoss import GptOssExpertsMxfp4
from .experts import Experts4bit, ExpertsNbit
from .lora import ExpertsLoRA, _epilogue

_PATH = {"auto": N.PATH_AUTO, "gemv": N.PATH_GEMV, "mfma": N.PATH_MFMA}
_kernel_path = N.PATH_AUTO


def set_kernel_path(path: str) -> None:
    """Force the grouped-GEMM kernel family ("auto" | "gemv" | "mfma"); for tests and benchmarks."""
    global _kernel_path
    _kernel_path = _PATH[path]


def fast_available() -> bool:
    """True iff the MI355X kernel library loads and a HIP device is up (``fast.py:66-72``)."""
    return N.available() and torch.cuda.is_available()


def _eligible(mod) -> Optional[str]:
    """None if ``mod`` can take the fast path, else the reason not (``fast.py:75-97``)."""
    if getattr(mod, "_e4b_mxfp4_arena", False):
        return ("storage is MXFP4 (arena), which the NF4 grouped kernel cannot read -- "
                "the MXFP4 forward is wired by nvme_experts and needs no patch here")
    if getattr(mod, "bits", None) != 4 or getattr(mod, "quant_type", None) != "nf4":
        return "storage is not nf4-4bit"
    if getattr(mod, "blocksize", None) != 64:
        return f"blocksize {getattr(mod, 'blocksize', None)} != 64"
    n1, k1 = mod._gate_up_shape
    n2, k2 = mod._down_shape
    if k1 % 64 or k2 % 64:
        return "K not divisible by 64"
    if not mod.gate_up_proj.is_cuda:
        return "storage not on CUDA"
    return None


def _eligible_mxfp4(mod) -> Optional[str]:
    n1, k1 = mod._gate_up_shape
    n2, k2 = mod._down_shape
    if k1 % 64 or k2 % 64:
        return "K not divisible by 64"
    if not mod.gate_up_proj.is_cuda:
        return "storage not on CUDA"
    return None


# ------------------------------------------------------------------- kernel descriptors


_SOURCES = ("gate_up_proj", "gate_up_absmax", "down_proj", "down_absmax", "code")
_SOURCES_DQ = _SOURCES + ("gate_up_absmax2", "gate_up_absmax_offset", "down_absmax2", "down_absmax_offset", "code2")


def _module_tensor(mod, name):
    """``getattr(mod, name)`` for a buffer or parameter, read from the module's own dicts (per
    call this skips ``nn.Module.__getattr__``, about 0.2 us a lookup on an eager decode call)."""
    t = mod._buffers.get(name)
    if t is None:
        t = mod._parameters.get(name)
    return t if t is not None else getattr(mod, name)


def _qweight_sources(mod):
    names = _SOURCES_DQ if getattr(mod, "compress_statistics", False) else _SOURCES
    return [_module_tensor(mod, n) for n in names]


# Kernel descriptors per module, outside the module itself: a module's own state must stay
# deep-copyable and picklable (the descriptors hold ctypes structs with raw pointers), and an
# entry disappears with its module.
_DESC_CACHE: "weakref.WeakKeyDictionary[torch.nn.Module, dict]" = weakref.WeakKeyDictionary()


def _cached_descriptors(mod, tag, sources, build):
    """``build()``'s result for ``mod``, rebuilt whenever a source tensor's storage moves
    (address: a new tensor, or a ``.data`` swap) or is updated in place (version counter, which
    ``load_state_dict`` copies bump). The descriptors hold the module's own tensor objects, so
    equal addresses and versions mean the pointers they carry are still those of the current
    storage. Inference tensors carry no version counter and cannot be written in place outside
    inference mode: they are keyed on their address alone, so an in-place write into one inside
    ``torch.inference_mode`` is not seen (``disable_fast`` / ``enable_fast``, or a new tensor,
    drops the entry)."""
    key = tuple([(t.data_ptr(), -1 if t.is_inference() else t._version) for t in sources])
    per_mod = _DESC_CACHE.setdefault(mod, {})
    hit = per_mod.get(tag)
    if hit is not None and hit[0] == key:
        return hit[1]
    value = build()
    per_mod[tag] = (key, value)
    return value


def _drop_descriptors(mod) -> None:
    """Forget ``mod``'s cached descriptors (and the weight tensors they keep alive)."""
    _DESC_CACHE.pop(mod, None)


def _qweights(mod):
    """(gate_up, down) kernel descriptors of an NF4 ``ExpertsNbit``, cached per module."""
    return _cached_descriptors(mod, "nf4", _qweight_sources(mod), lambda: _build_qweights(mod))


def _build_qweights(mod):
    E = mod.num_experts
    n1, k1 = mod._gate_up_shape
    n2, k2 = mod._down_shape
    if getattr(mod, "compress_statistics", False):
        w1 = ops.nf4_dq_qweight(mod.gate_up_proj, mod.gate_up_absmax, mod.gate_up_absmax2, mod.gate_up_absmax_offset,
                                mod.code, mod.code2, n1, k1, num_experts=E)
        w2 = ops.nf4_dq_qweight(mod.down_proj, mod.down_absmax, mod.down_absmax2, mod.down_absmax_offset,
                                mod.code, mod.code2, n2, k2, num_experts=E)
    else:
        w1 = ops.nf4_qweight(mod.gate_up_proj, mod.gate_up_absmax, mod.code, n1, k1, num_experts=E)
        w2 = ops.nf4_qweight(mod.down_proj, mod.down_absmax, mod.code, n2, k2, num_experts=E)
    return w1, w2


# Up to this many tokens the fused forward runs the decode / GEMV kernels, which never read the
# per-expert weight exponents (the C side's fp16 matrix-core mode starts above it).
_SHIFT_FREE_TOKENS = 4


def _for_tokens(descs, tokens):
    """The (gate_up, down) descriptors a call of ``tokens`` tokens needs: above
    ``_SHIFT_FREE_TOKENS`` with the per-expert exponents that let the matrix-core GEMMs run on
    fp16 operands, computed on the first such call and kept with the cached descriptors (once per
    weight version); below it as they are, so decode calls never launch the exponent kernels."""
    if tokens <= _SHIFT_FREE_TOKENS:
        return descs
    for qw in descs:
        if qw.shift is None:
            ops.with_weight_shift(qw)
    return descs


def _mxfp4_qweights(mod, cd):
    """(gate_up, down) descriptors of a ``GptOssExpertsMxfp4`` with its biases in the compute
    dtype ``cd``, cached per module like the NF4 ones (the bias casts included)."""
    E = mod.num_experts
    n1, k1 = mod._gate_up_shape
    n2, k2 = mod._down_shape

    def build():
        w1 = ops.mxfp4_qweight(mod.gate_up_proj, mod.gate_up_absmax, n1, k1, num_experts=E,
                               bias=mod.gate_up_bias.to(cd))
        w2 = ops.mxfp4_qweight(mod.down_proj, mod.down_absmax, n2, k2, num_experts=E, bias=mod.down_bias.to(cd))
        return w1, w2

    srcs = [mod.gate_up_proj, mod.gate_up_absmax, mod.gate_up_bias, mod.down_proj, mod.down_absmax, mod.down_bias]
    return _cached_descriptors(mod, ("mxfp4", cd), srcs, build)


def _fused_epilogue(base):
    """(epilogue code, limit) the kernel can apply for this base, or None when only the base's own
    Python epilogue reproduces it (a custom ``_apply_gate`` or activation)."""
    hook = getattr(base, "_apply_gate", None)
    if hook is not None:
        if isinstance(base, _DeepseekV4ForwardMixin) and type(base)._apply_gate is _DeepseekV4ForwardMixin._apply_gate:
            return N.EPI_CLAMP_SWIGLU, float(base.limit)
        return None
    if base.act_fn is not F.silu:
        return None
    return (N.EPI_SWIGLU if base.has_gate else N.EPI_ACT), 0.0


def _wants_reference(mod, hidden_states) -> bool:
    return torch.is_grad_enabled() and (hidden_states.requires_grad or any(p.requires_grad for p in mod.parameters()))


# ------------------------------------------------------------------------ fused forwards


def fused_experts_forward(mod, hidden_states, top_k_index, top_k_weights):
    """Fused inference forward of a bare ``ExpertsNbit`` (``fast.py:100-160``)."""
    if _wants_reference(mod, hidden_states):
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    compute_dtype = mod.compute_dtype if mod.compute_dtype is not None else hidden_states.dtype
    if compute_dtype not in (torch.bfloat16, torch.float16):
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    if _module_tensor(mod, "gate_up_proj").numel() == 0 or _module_tensor(mod, "down_proj").numel() == 0:
        _drop_descriptors(mod)  # the evicted weights must not stay alive through the cache
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    return _bare_forward(mod, hidden_states, top_k_index, top_k_weights, compute_dtype)


def _bare_forward(mod, hidden_states, top_k_index, top_k_weights, compute_dtype):
    """The fused forward of a bare NF4 base once the fallbacks are ruled out."""
    input_dtype = hidden_states.dtype
    x = hidden_states if input_dtype == compute_dtype else hidden_states.to(compute_dtype)
    tokens = x.shape[0]
    k = top_k_index.shape[1]
    hidden = mod._down_shape[0]
    if tokens == 0:
        return torch.zeros(0, hidden, dtype=input_dtype, device=x.device)
    w1, w2 = _for_tokens(_qweights(mod), tokens)
    epi = _fused_epilogue(mod)
    if epi is not None:
        code, limit = epi
        return ops.moe_forward(x, top_k_index, top_k_weights, w1, w2, code, input_dtype, limit=limit,
                               path=_kernel_path)
    # custom epilogue: unfused GEMMs around the base's own Python epilogue
    M = tokens * k
    rb = ops.route(top_k_index, mod.num_experts)
    up = ops.grouped_gemm(x, w1, rb, tokens, M, N.EPI_NONE, gather_k=k, path=_kernel_path, out_dtype=torch.float32)
    h = _epilogue(mod, up).to(compute_dtype).contiguous()
    down = ops.grouped_gemm(h, w2, rb, tokens, M, N.EPI_NONE, path=_kernel_path, out_dtype=torch.float32)
    return ops.combine(down, rb, top_k_weights, tokens, k, input_dtype)


def fused_experts_lora_forward(mod, hidden_states, top_k_index, top_k_weights):
    """Fused inference forward of an ``ExpertsLoRA`` (``fast.py:163-257``), with no device->host
    synchronisation (the reference slices its expert groups in Python after a ``.tolist()``).

    With a kernel epilogue (SwiGLU, clamped SwiGLU, SiLU) the whole layer is one C-ABI call,
    ``e4b_moe_lora_forward``: up to 8 tokens add the low-rank deltas inside the decode GEMVs
    (four launches), larger batches run the grouped GEMMs with every expert group's delta added
    on the device. A custom activation keeps the base's own Python epilogue between the grouped
    GEMMs, the deltas applied by ``e4b_lora_delta``. Either way the deltas stay fp32 until h and
    the combined output are rounded (fewer rounding points than the reference's compute-dtype
    casts, ``lora.py:256``, as for the base path)."""
    base = mod.base
    if _wants_reference(mod, hidden_states):
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    if mod.training:
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    compute_dtype = base.compute_dtype if base.compute_dtype is not None else hidden_states.dtype
    if compute_dtype not in (torch.bfloat16, torch.float16):
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    if base.gate_up_proj.numel() == 0 or base.down_proj.numel() == 0:
        _drop_descriptors(base)  # the evicted weights must not stay alive through the cache
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    if mod._adapter_is_zero():
        # the adapter contributes exactly nothing (both B zero): the base's own fused forward,
        # one call, as the reference's delegation to an accelerated base (lora.py:181-214). The
        # verdict costs one sync on the first call and is cached until train() / a state load.
        return _bare_forward(base, hidden_states, top_k_index, top_k_weights, compute_dtype)

    input_dtype = hidden_states.dtype
    x = hidden_states if input_dtype == compute_dtype else hidden_states.to(compute_dtype)
    tokens = x.shape[0]
    k = top_k_index.shape[1]
    hidden = base._down_shape[0]
    if tokens == 0:
        return torch.zeros(0, hidden, dtype=input_dtype, device=x.device)
    E = base.num_experts
    M = tokens * k
    w1, w2 = _for_tokens(_qweights(base), tokens)
    r = mod.gate_up_lora_A.shape[1]
    if r > 64 or x.shape[1] % 8 or base._down_shape[1] % 8:  # beyond the delta kernel's limits
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    epi = _fused_epilogue(base)
    if epi is not None:
        return ops.moe_lora_forward(x, top_k_index, top_k_weights, w1, w2,
                                    (mod.gate_up_lora_A, mod.gate_up_lora_B), (mod.down_lora_A, mod.down_lora_B),
                                    mod.scaling, epi[0], input_dtype, limit=epi[1], path=_kernel_path)
    # a custom activation: the base's own Python epilogue between the grouped GEMMs
    rb = ops.route(top_k_index, E)
    up = ops.grouped_gemm(x, w1, rb, tokens, M, N.EPI_NONE, gather_k=k, path=_kernel_path, out_dtype=torch.float32)
    ops.lora_delta(x, rb, M, E, mod.gate_up_lora_A, mod.gate_up_lora_B, mod.scaling, up, gather_k=k,
                   delta_dtype=torch.float32)
    h = _epilogue(base, up).to(compute_dtype).contiguous()
    down = ops.grouped_gemm(h, w2, rb, tokens, M, N.EPI_NONE, path=_kernel_path, out_dtype=torch.float32)
    ops.lora_delta(h, rb, M, E, mod.down_lora_A, mod.down_lora_B, mod.scaling, down, delta_dtype=torch.float32)
    return ops.combine(down, rb, top_k_weights, tokens, k, input_dtype)


def fused_mxfp4_forward(mod, hidden_states, top_k_index, top_k_weights):
    """Fused inference forward of a ``GptOssExpertsMxfp4``: MXFP4 decode in both GEMMs, gate_up
    bias + clamped GLU fused into the first, down bias into the second, the deterministic
    combine (the grouped path of ``hot_residency.py:72-80`` / ``nvme_experts.py:805-868``)."""
    if _wants_reference(mod, hidden_states):
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    cd = mod.compute_dtype if mod.compute_dtype is not None else hidden_states.dtype
    if mod.gate_up_proj.numel() == 0 or mod.down_proj.numel() == 0:
        _drop_descriptors(mod)
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    if cd not in (torch.bfloat16, torch.float16):
        return mod._e4b_fast_ref(hidden_states, top_k_index, top_k_weights)
    input_dtype = hidden_states.dtype
    x = hidden_states.to(cd)
    if x.shape[0] == 0:
        return torch.zeros(0, mod.hidden_dim, dtype=input_dtype, device=x.device)
    w1, w2 = _mxfp4_qweights(mod, cd)
    return ops.moe_forward(x, top_k_index, top_k_weights, w1, w2, N.EPI_GPTOSS, input_dtype, alpha=mod.alpha,
                           limit=mod.limit, path=_kernel_path)


# ------------------------------------------------------------------------- patching


def enable_fast(model, verbose: bool = False) -> int:
    """Patch every eligible expert module under ``model`` (or ``model`` itself); returns the count
    (``fast.py:281-411``)."""
    stock_forwards = {ExpertsNbit.forward, Experts4bit.forward}
    mods = list(model.modules()) if hasattr(model, "modules") else [model]
    patched = 0

    wrapped_bases = {id(m.base) for m in mods if isinstance(m, ExpertsLoRA)}
    for mod in mods:
        if not isinstance(mod, ExpertsLoRA):
            continue
        if type(mod).forward is not ExpertsLoRA.forward:
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: custom forward")
            continue
        if not isinstance(mod.base, ExpertsNbit):
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: base {type(mod.base).__name__} is not an ExpertsNbit")
            continue
        reason = _eligible(mod.base)
        if reason is not None:
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: {reason}")
            continue
        if type(mod.base).forward not in stock_forwards and not hasattr(mod.base, "_apply_gate"):
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: base {type(mod.base).__name__} has a custom forward")
            continue
        if hasattr(mod, "_e4b_fast_ref"):
            continue
        mod._e4b_fast_ref = mod.forward
        mod.forward = fused_experts_lora_forward.__get__(mod)
        patched += 1

    for mod in mods:
        if isinstance(mod, GptOssExpertsMxfp4):
            if id(mod) in wrapped_bases:
                continue
            reason = _eligible_mxfp4(mod)
            if reason is not None:
                if verbose:
                    print(f"[e4b.fast] skip {type(mod).__name__}: {reason}")
                continue
            if hasattr(mod, "_e4b_fast_ref"):
                continue
            mod._e4b_fast_ref = mod.forward
            mod.forward = fused_mxfp4_forward.__get__(mod)
            patched += 1
            continue
        if not isinstance(mod, ExpertsNbit):
            continue
        if id(mod) in wrapped_bases:
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: wrapped by a patched ExpertsLoRA "
                      "(its forward is never called)")
            continue
        if type(mod).forward not in stock_forwards and not hasattr(mod, "_apply_gate"):
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: custom forward")
            continue
        reason = _eligible(mod)
        if reason is not None:
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: {reason}")
            continue
        skip = None
        for attr, what in (("_hot_residency", "hot_residency"), ("_e4b_cold_ref", "cold engine"),
                           ("_e4b_pipe_ref", "pipelined residency"), ("_e4b_mxfp4_ref", "mxfp4 NVMe residency")):
            if hasattr(mod, attr):
                skip = what
                break
        if skip is not None:
            if verbose:
                print(f"[e4b.fast] skip {type(mod).__name__}: {skip} enabled -- disable it first")
            continue
        if hasattr(mod, "_e4b_fast_ref"):
            continue
        mod._e4b_fast_ref = mod.forward
        mod.forward = fused_experts_forward.__get__(mod)
        patched += 1

    if patched and getattr(model, "training", False):
        import warnings

        warnings.warn(
            f"[e4b.fast] model is in TRAINING mode: fused_experts_lora_forward falls back to the reference "
            f"path while `training` is set, so all {patched} patch(es) will be bypassed and the fused kernel "
            "will not run. Call model.eval() before inference.",
            RuntimeWarning, stacklevel=2)
    return patched


def disable_fast(model) -> int:
    """Undo :func:`enable_fast`; returns the number of modules restored (``fast.py:414-423``)."""
    mods = model.modules() if hasattr(model, "modules") else [model]
    restored = 0
    for mod in mods:
        if hasattr(mod, "_e4b_fast_ref"):
            mod.forward = mod._e4b_fast_ref
            del mod._e4b_fast_ref
            restored += 1
        _drop_descriptors(mod)
    return restored
