"""N-bit fused-expert storage modules: ``ExpertsNbit`` and its 4-bit specialisation ``Experts4bit``.

The same constructor, buffers, ``state_dict`` keys and ``_extra_state`` contract as the
reference (``experts4bit_qlora/_vendor/experts.py:123-530``), so checkpoints move between the
two unchanged:

* ``gate_up_proj`` / ``down_proj``: frozen ``nn.Parameter`` uint8 ``[E, out*in/2]`` (4-bit, first
  value of a pair in the high nibble), ``[E, out*in]`` (8-bit codes) or the weights themselves
  (16-bit passthrough); each expert's ``[out, in]`` matrix is flattened row-major.
* ``gate_up_absmax`` / ``down_absmax``: fp32 ``[E, out*in/blocksize]`` (``None`` for passthrough).
* ``code``: the non-persistent codebook.
* ``_extra_state``: schema 1, ``quant_type, blocksize, has_gate, num_experts, hidden_dim,
  intermediate_dim``, validated on load; legacy checkpoints without it load unvalidated.

Extension beyond the reference: ``compress_statistics=True`` (4-bit only) stores the absmax
double-quantized -- uint8 codes in ``*_absmax``, fp32 ``*_absmax2`` per 256 blocks and a
per-expert fp32 ``*_absmax_offset`` -- which the fused kernels decode on the fly.

``forward`` is the reference per-expert loop (``_vendor/experts.py:468-516``): it is the
training path (the recompute-in-backward projection), the fallback the fused forward hands
back to, and the accuracy anchor the fused path is graded against. On a HIP device the
4-bit dequantize inside it runs the library's bit-exact ``e4b_dequant`` kernel.
"""
from __future__ import annotations

import functools
from collections.abc import Callable
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F_nn

from . import quant as Q

_SCHEME_BITS = {"nf4": 4, "fp4": 4, "int8": 8, "fp8": 8, "bf16": 16, "fp16": 16}
_PASSTHROUGH_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}
_EXTRA_STATE_SCHEMA = 1
_QUANT_TYPE_ALIASES = {"bfloat16": "bf16", "float16": "fp16"}


def normalize_quant_type(quant_type, allowed: tuple = tuple(_SCHEME_BITS)) -> str:
    """Canonicalise a storage-scheme name (case/whitespace-insensitive, torch-dtype longhands
    accepted); raises ``ValueError`` naming the allowed set. Same contract as
    ``_vendor/experts.py:42-58``."""
    if not isinstance(quant_type, str):
        raise ValueError(f"quant_type must be one of {allowed}, got {type(quant_type).__name__}")
    q = quant_type.strip().lower()
    q = _QUANT_TYPE_ALIASES.get(q, q)
    if q not in allowed:
        hint = f" (normalized from {quant_type!r})" if q != quant_type else ""
        raise ValueError(f"quant_type must be one of {allowed}, got {q!r}{hint}")
    return q


def _build_code(quant_type: str, device) -> Optional[torch.Tensor]:
    device = "cpu" if device is None else device
    if quant_type in ("nf4", "fp4"):
        return Q.code_4bit(quant_type, device=device)
    if quant_type == "int8":
        return Q.dynamic_map().to(device)
    if quant_type == "fp8":
        return Q.fp8_map().to(device)
    return None


class _FrozenLinearRecomputeBackward(torch.autograd.Function):
    """``F.linear`` against a frozen dequantized weight, re-dequantized in backward (the weight
    is never saved as an activation). Same contract as ``_vendor/experts.py:80-120``."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, dequant_fn: Callable[[], torch.Tensor]) -> torch.Tensor:
        ctx.dequant_fn = dequant_fn
        return F_nn.linear(x, dequant_fn())

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        grad_x = None
        if ctx.needs_input_grad[0]:
            try:
                weight = ctx.dequant_fn()
            except Exception as e:
                packed = ctx.dequant_fn.args[0] if getattr(ctx.dequant_fn, "args", None) else None
                if isinstance(packed, torch.Tensor) and packed.numel() == 0:
                    raise RuntimeError(
                        "backward re-dequantization read an offload-evicted expert (0-element "
                        "placeholder); offloaded training needs gradient checkpointing so the "
                        "recompute re-stages the layer before its backward runs"
                    ) from e
                raise
            grad_x = grad_output @ weight
        return grad_x, None


class ExpertsNbit(nn.Module):
    """Low-bit quantized storage for fused MoE expert weights (``[E, out, in]`` stacks).

    Args mirror the reference: ``num_experts``, ``hidden_dim``, ``intermediate_dim``,
    ``has_gate`` (SwiGLU-packed gate_up), ``activation`` (default SiLU), ``compute_dtype``,
    ``quant_type`` (nf4/fp4/int8/fp8/bf16/fp16), ``blocksize``, ``device``; plus
    ``compress_statistics`` (4-bit double-quantized absmax).
    """

    _ALLOWED_QUANT_TYPES: tuple = tuple(_SCHEME_BITS)
    _EXTRA_STATE_FIELDS = ("quant_type", "blocksize", "has_gate", "num_experts", "hidden_dim", "intermediate_dim")

    def __init__(self, num_experts: int, hidden_dim: int, intermediate_dim: int, has_gate: bool = True,
                 activation: Optional[Callable[[torch.Tensor], torch.Tensor]] = None,
                 compute_dtype: Optional[torch.dtype] = None, quant_type: str = "nf4", blocksize: int = 64,
                 device=None, compress_statistics: bool = False):
        super().__init__()
        quant_type = normalize_quant_type(quant_type, allowed=type(self)._ALLOWED_QUANT_TYPES)
        self.bits = _SCHEME_BITS[quant_type]
        if self.bits < 16:
            for name, in_features in (("hidden_dim", hidden_dim), ("intermediate_dim", intermediate_dim)):
                if in_features % blocksize != 0:
                    raise ValueError(
                        f"{name} ({in_features}) must be divisible by blocksize ({blocksize}) "
                        "so per-expert quantization blocks align with expert boundaries")
        if compress_statistics and self.bits != 4:
            raise ValueError("compress_statistics (double-quant absmax) applies to the 4-bit schemes only")
        self.num_experts = num_experts
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.has_gate = has_gate
        self.act_fn = activation if activation is not None else F_nn.silu
        self.compute_dtype = compute_dtype
        self.quant_type = quant_type
        self.blocksize = blocksize
        self.compress_statistics = bool(compress_statistics)

        gate_up_out = 2 * intermediate_dim if has_gate else intermediate_dim
        self._gate_up_shape = (gate_up_out, hidden_dim)
        self._down_shape = (hidden_dim, intermediate_dim)
        gu_numel = gate_up_out * hidden_dim
        dn_numel = hidden_dim * intermediate_dim

        if self.bits == 16:
            sd = _PASSTHROUGH_DTYPES[quant_type]
            gu = torch.empty(num_experts, gu_numel, dtype=sd, device=device)
            dn = torch.empty(num_experts, dn_numel, dtype=sd, device=device)
        else:
            per = 2 if self.bits == 4 else 1
            gu = torch.empty(num_experts, gu_numel // per, dtype=torch.uint8, device=device)
            dn = torch.empty(num_experts, dn_numel // per, dtype=torch.uint8, device=device)
        self.gate_up_proj = nn.Parameter(gu, requires_grad=False)
        self.down_proj = nn.Parameter(dn, requires_grad=False)

        if self.bits < 16:
            adt = torch.uint8 if self.compress_statistics else torch.float32
            self.register_buffer("gate_up_absmax", torch.empty(num_experts, gu_numel // blocksize, dtype=adt, device=device))
            self.register_buffer("down_absmax", torch.empty(num_experts, dn_numel // blocksize, dtype=adt, device=device))
        else:
            self.register_buffer("gate_up_absmax", None)
            self.register_buffer("down_absmax", None)
        if self.compress_statistics:
            nb2 = lambda numel: -(-(numel // blocksize) // 256)  # noqa: E731
            self.register_buffer("gate_up_absmax2", torch.empty(num_experts, nb2(gu_numel), device=device))
            self.register_buffer("down_absmax2", torch.empty(num_experts, nb2(dn_numel), device=device))
            self.register_buffer("gate_up_absmax_offset", torch.empty(num_experts, device=device))
            self.register_buffer("down_absmax_offset", torch.empty(num_experts, device=device))
            self.register_buffer("code2", Q.dynamic_map().to(device if device is not None else "cpu"),
                                 persistent=False)
        self.register_buffer("code", _build_code(quant_type, device), persistent=False)

    # ------------------------------------------------------------------ state_dict contract
    def get_extra_state(self) -> dict:
        state = {"schema": _EXTRA_STATE_SCHEMA}
        state.update({k: getattr(self, k) for k in self._EXTRA_STATE_FIELDS})
        if self.compress_statistics:
            state["compress_statistics"] = True
        return state

    def set_extra_state(self, state) -> None:
        if state is None:
            return
        if not isinstance(state, dict) or not isinstance(state.get("schema"), int):
            raise ValueError(f"unrecognized ExpertsNbit extra state: {type(state).__name__}")
        if state["schema"] > _EXTRA_STATE_SCHEMA:
            raise ValueError(
                f"checkpoint carries ExpertsNbit metadata schema {state['schema']}; this build "
                f"understands <= {_EXTRA_STATE_SCHEMA}")
        fields = self._EXTRA_STATE_FIELDS + ("compress_statistics",)
        bad = {k: (state[k], getattr(self, k)) for k in fields if k in state and state[k] != getattr(self, k)}
        if self.compress_statistics and not state.get("compress_statistics", False):
            bad["compress_statistics"] = (False, True)
        if bad:
            detail = ", ".join(f"{k}: checkpoint={c!r} vs module={m!r}" for k, (c, m) in bad.items())
            raise ValueError("checkpoint/module config mismatch -- re-instantiate the module with the "
                             f"checkpoint's construction arguments ({detail})")

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        state_dict.setdefault(prefix + "_extra_state", None)
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)

    # ------------------------------------------------------------------------ construction
    @classmethod
    def from_float(cls, gate_up_proj: torch.Tensor, down_proj: torch.Tensor, has_gate: bool = True,
                   activation: Optional[Callable[[torch.Tensor], torch.Tensor]] = None,
                   compute_dtype: Optional[torch.dtype] = None, quant_type: str = "nf4", blocksize: int = 64,
                   compress_statistics: bool = False) -> "ExpertsNbit":
        """Quantize ``[E, gate_up_out, hidden]`` and ``[E, hidden, inter]`` stacks into a module
        on the inputs' device (same layout checks as ``_vendor/experts.py:329-396``)."""
        if gate_up_proj.dim() != 3 or down_proj.dim() != 3:
            raise ValueError("gate_up_proj and down_proj must be 3D [num_experts, out, in] tensors")
        num_experts, gate_up_out, hidden_dim = gate_up_proj.shape
        intermediate_dim = down_proj.shape[2]
        expected = 2 * intermediate_dim if has_gate else intermediate_dim
        if down_proj.shape[0] != num_experts or down_proj.shape[1] != hidden_dim or gate_up_out != expected:
            raise ValueError(
                f"inconsistent expert stacks for has_gate={has_gate}: expected gate_up_proj "
                f"[num_experts, {'2*intermediate' if has_gate else 'intermediate'}, hidden] and down_proj "
                f"[num_experts, hidden, intermediate] (layout [num_experts, out, in]), got gate_up_proj "
                f"{tuple(gate_up_proj.shape)} vs down_proj {tuple(down_proj.shape)} -- is one of them "
                "transposed / stored [num_experts, in, out]?")
        module = cls(num_experts, hidden_dim, intermediate_dim, has_gate=has_gate, activation=activation,
                     compute_dtype=compute_dtype if compute_dtype is not None else gate_up_proj.dtype,
                     quant_type=quant_type, blocksize=blocksize, device=gate_up_proj.device,
                     compress_statistics=compress_statistics)
        for name, w in (("gate_up", gate_up_proj), ("down", down_proj)):
            packed, absmax = module._quantize_stack(w)
            setattr(module, f"{name}_proj", nn.Parameter(packed, requires_grad=False))
            if module.compress_statistics:
                q, a2, off = Q.double_quant(absmax, code2=module.code2)
                setattr(module, f"{name}_absmax", q)
                setattr(module, f"{name}_absmax2", a2)
                setattr(module, f"{name}_absmax_offset", off)
            else:
                setattr(module, f"{name}_absmax", absmax)
        return module

    def _quantize_stack(self, weights: torch.Tensor):
        """``[E, out, in]`` -> (packed ``[E, ...]``, absmax ``[E, blocks]`` or ``None``). Blocks never
        straddle experts, so the whole stack quantizes in one pass."""
        E = weights.shape[0]
        flat = weights.reshape(E, -1)
        if self.bits == 16:
            return flat.to(_PASSTHROUGH_DTYPES[self.quant_type]).contiguous(), None
        if self.bits == 4:
            packed, absmax = Q.quantize_4bit(flat.float(), self.quant_type, self.blocksize)
            return packed.contiguous(), absmax.contiguous()
        q, absmax = Q.quantize_blocks(flat.float(), self.code.to(flat.device), self.blocksize)
        return q.contiguous(), absmax.contiguous()

    # ----------------------------------------------------------------------------- dequant
    def _absmax_parts(self, absmax: torch.Tensor):
        """(absmax2, offset) buffers that belong with a double-quantized absmax buffer."""
        if absmax is self.gate_up_absmax:
            return self.gate_up_absmax2, self.gate_up_absmax_offset
        if absmax is self.down_absmax:
            return self.down_absmax2, self.down_absmax_offset
        raise ValueError("double-quantized absmax must be this module's gate_up_absmax or down_absmax")

    def _dequantize_expert(self, packed: torch.Tensor, absmax: Optional[torch.Tensor], shape: tuple[int, int],
                           expert_idx, dtype: torch.dtype) -> torch.Tensor:
        """Dequantize one expert's ``[out, in]`` weight (``_vendor/experts.py:428-457``).

        4-bit: ``dtype(code[nib] * absmax)`` bit-exactly -- on a HIP device through the library's
        ``e4b_dequant`` kernel (it raises if the library is missing), on the CPU in torch.
        ``expert_idx`` may be an int or a 0-d device tensor (no host sync either way).
        """
        if self.bits == 16:
            return packed[expert_idx].reshape(shape).to(dtype)
        if self.bits == 8:
            a = absmax[expert_idx].reshape(-1, 1)
            vals = self.code.to(packed.device)[packed[expert_idx].long()].reshape(-1, self.blocksize)
            return (vals * a).reshape(shape).to(dtype)
        pk = packed[expert_idx]
        if self.compress_statistics:
            a2, off = self._absmax_parts(absmax)
            q, a2e, offe = absmax[expert_idx], a2[expert_idx], off[expert_idx]
        else:
            am = absmax[expert_idx]
        if pk.is_cuda:
            from . import ops

            n, k = shape
            if self.blocksize != 64:
                raise NotImplementedError("the HIP dequant kernel decodes blocksize 64 (the reference's default)")
            if self.compress_statistics:
                qw = ops.nf4_dq_qweight(pk.reshape(1, -1), q.reshape(1, -1), a2e.reshape(1, -1), offe.reshape(1),
                                        self.code, self.code2, n, k, num_experts=1)
            else:
                qw = ops.nf4_qweight(pk.reshape(1, -1), am.reshape(1, -1), self.code, n, k, num_experts=1)
            return ops.dequant(qw, 0, 1, dtype=dtype)[0]
        if self.compress_statistics:
            am = Q.dequant_absmax(q.reshape(1, -1), a2e.reshape(1, -1), offe.reshape(1), self.code2)[0]
        return Q.dequant_4bit_torch(pk, am, self.code, shape, self.blocksize, dtype)

    def _project(self, packed, absmax, shape, expert_idx, x, compute_dtype):
        """One expert projection: dequantize + ``linear``, re-dequantizing in backward."""
        dequant_fn = functools.partial(self._dequantize_expert, packed, absmax, shape, expert_idx, compute_dtype)
        return _FrozenLinearRecomputeBackward.apply(x, dequant_fn)

    # ----------------------------------------------------------------------------- forward
    def forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor) -> torch.Tensor:
        """Reference per-expert loop (``_vendor/experts.py:468-516``)."""
        input_dtype = hidden_states.dtype
        compute_dtype = self.compute_dtype if self.compute_dtype is not None else hidden_states.dtype
        hidden_states = hidden_states.to(compute_dtype)
        final_hidden_states = torch.zeros_like(hidden_states, dtype=torch.float32)
        with torch.no_grad():
            expert_mask = F_nn.one_hot(top_k_index, num_classes=self.num_experts).permute(2, 1, 0)
            expert_hit = torch.greater(expert_mask.sum(dim=(-1, -2)), 0).nonzero(as_tuple=False).view(-1)
        for expert_idx in expert_hit:
            top_k_pos, token_idx = torch.where(expert_mask[expert_idx])
            current_state = hidden_states[token_idx]
            proj = self._project(self.gate_up_proj, self.gate_up_absmax, self._gate_up_shape, expert_idx,
                                 current_state, compute_dtype)
            if self.has_gate:
                gate, up = proj.chunk(2, dim=-1)
                current_hidden = self.act_fn(gate) * up
            else:
                current_hidden = self.act_fn(proj)
            current_hidden = self._project(self.down_proj, self.down_absmax, self._down_shape, expert_idx,
                                           current_hidden, compute_dtype)
            current_hidden = current_hidden * top_k_weights[token_idx, top_k_pos, None]
            final_hidden_states.index_add_(0, token_idx, current_hidden.to(final_hidden_states.dtype))
        return final_hidden_states.to(input_dtype)


class Experts4bit(ExpertsNbit):
    """4-bit (``nf4`` / ``fp4``) quantized storage for fused MoE expert weights; see
    :class:`ExpertsNbit` (``_vendor/experts.py:519-530``)."""

    _ALLOWED_QUANT_TYPES = ("nf4", "fp4")
