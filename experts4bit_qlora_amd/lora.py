"""Per-expert LoRA over a frozen expert base, and the base-owned epilogue hook.

``ExpertsLoRA`` keeps the reference's parameters, forward contract and delegation rules
(``experts4bit_qlora/lora.py:131-460``): ``gate_up_lora_A [E, r, hidden]``, ``gate_up_lora_B
[E, gate_up_out, r]``, ``down_lora_A [E, r, inter]``, ``down_lora_B [E, hidden, r]``, B zero-init so
an untrained adapter is exactly the base; the low-rank delta lands BEFORE the activation.

The reference's optional single-row route through bitsandbytes' ``gemv_4bit``
(``lora.py:258-327``) is not reproduced: bitsandbytes is not part of this build, and the
inference fast path replaces this whole forward (``enable_fast``). ``_use_infer_gemv`` therefore
always answers False and the dequantize path serves single rows.
"""
from __future__ import annotations

import os

import torch
import torch.nn as nn
import torch.nn.functional as F


def _decode_fastpath_enabled() -> bool:
    """Single-token decode fast-path kill-switch (``E4B_DECODE_FASTPATH=0``); default on."""
    return os.environ.get("E4B_DECODE_FASTPATH", "1") != "0"


def _epilogue(base, proj):
    """The base's own activation (``lora.py:102-128``): ``base._apply_gate`` when the base has
    one (DeepSeek-V4's clamped SwiGLU, computed in fp32 and cast back), else
    ``act_fn(gate) * up`` over the two halves, else ``act_fn(proj)``."""
    hook = getattr(base, "_apply_gate", None)
    if hook is not None:
        out = hook(proj)
        return out if out.dtype == proj.dtype else out.to(proj.dtype)
    if base.has_gate:
        gate, up = proj.chunk(2, dim=-1)
        return base.act_fn(gate) * up
    return base.act_fn(proj)


class ExpertsLoRA(nn.Module):
    """Per-expert LoRA adapters over a frozen :class:`Experts4bit` / :class:`ExpertsNbit` base."""

    def __init__(self, base, r: int = 8, alpha: int = 16, dtype: torch.dtype = torch.float32):
        super().__init__()
        self.base = base
        for p in self.base.parameters():
            p.requires_grad_(False)
        if r < 1:
            raise ValueError(
                f"ExpertsLoRA needs rank r >= 1, got r={r}. For 'no adapter', keep an ordinary rank and "
                "leave the adapter untrained: B is zero-initialised, so the delta is identically zero.")
        self.r = r
        self.scaling = alpha / r
        self._delegate_ok = None
        num_experts = base.num_experts
        gate_up_out, hidden = base._gate_up_shape
        _, intermediate = base._down_shape
        self.gate_up_lora_A = nn.Parameter(torch.empty(num_experts, r, hidden, dtype=dtype))
        self.gate_up_lora_B = nn.Parameter(torch.zeros(num_experts, gate_up_out, r, dtype=dtype))
        self.down_lora_A = nn.Parameter(torch.empty(num_experts, r, intermediate, dtype=dtype))
        self.down_lora_B = nn.Parameter(torch.zeros(num_experts, hidden, r, dtype=dtype))
        nn.init.normal_(self.gate_up_lora_A, std=1.0 / r)
        nn.init.normal_(self.down_lora_A, std=1.0 / r)

    def _delegate_to_base(self) -> bool:
        """Hand the whole forward to the base when the adapter provably contributes nothing and an
        engine is attached to the base (``lora.py:181-214``)."""
        if torch.is_grad_enabled() or self.training:
            return False
        base = self.base
        if (getattr(base, "_e4b_fast_ref", None) is None and getattr(base, "_e4b_pipe_ref", None) is None
                and getattr(base, "_e4b_hot_ref", None) is None):
            return False
        return self._adapter_is_zero()

    def _adapter_is_zero(self) -> bool:
        """Whether both B matrices are exactly zero (one sync, cached; reset on train()/load)."""
        cached = self._delegate_ok
        if cached is None:
            cached = bool(self.r == 0 or (not self.gate_up_lora_B.any().item() and not self.down_lora_B.any().item()))
            self._delegate_ok = cached
        return cached

    def _load_from_state_dict(self, *args, **kwargs):
        self._delegate_ok = None
        return super()._load_from_state_dict(*args, **kwargs)

    def train(self, mode: bool = True):
        self._delegate_ok = None
        return super().train(mode)

    def _lora(self, x: torch.Tensor, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
        """``scaling * (x @ A.T) @ B.T`` in the adapter dtype, cast back (``lora.py:251-256``)."""
        return (self.scaling * F.linear(F.linear(x.to(A.dtype), A), B)).to(x.dtype)

    def _use_infer_gemv(self, hidden_states: torch.Tensor) -> bool:
        return False

    def _base_project(self, packed, absmax, shape, expert_idx, x, compute_dtype, use_gemv):
        return self.base._project(packed, absmax, shape, expert_idx, x, compute_dtype)

    def forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor) -> torch.Tensor:
        """Reference forward (``lora.py:329-407``): per hit expert, base projection + low-rank
        delta, the base's epilogue, base projection + delta, router weight, fp32 ``index_add_``."""
        base = self.base
        input_dtype = hidden_states.dtype
        compute_dtype = base.compute_dtype if base.compute_dtype is not None else hidden_states.dtype
        hidden_states = hidden_states.to(compute_dtype)
        if self._delegate_to_base():
            return base(hidden_states, top_k_index, top_k_weights).to(input_dtype)
        use_infer_gemv = self._use_infer_gemv(hidden_states)
        if (hidden_states.shape[0] == 1 and not torch.is_grad_enabled() and not self.training
                and _decode_fastpath_enabled()):
            return self._forward_decode(hidden_states, top_k_index, top_k_weights, compute_dtype, use_infer_gemv,
                                        input_dtype)
        final_hidden_states = torch.zeros_like(hidden_states, dtype=torch.float32)
        with torch.no_grad():
            expert_mask = F.one_hot(top_k_index, num_classes=base.num_experts).permute(2, 1, 0)
            expert_hit = torch.greater(expert_mask.sum(dim=(-1, -2)), 0).nonzero(as_tuple=False).view(-1)
        for expert_idx in expert_hit:
            top_k_pos, token_idx = torch.where(expert_mask[expert_idx])
            x = hidden_states[token_idx]
            proj = self._base_project(base.gate_up_proj, base.gate_up_absmax, base._gate_up_shape, expert_idx, x,
                                      compute_dtype, False) + self._lora(
                x, self.gate_up_lora_A[expert_idx], self.gate_up_lora_B[expert_idx])
            current_hidden = _epilogue(base, proj)
            current_hidden = self._base_project(base.down_proj, base.down_absmax, base._down_shape, expert_idx,
                                                current_hidden, compute_dtype, False) + self._lora(
                current_hidden, self.down_lora_A[expert_idx], self.down_lora_B[expert_idx])
            current_hidden = current_hidden * top_k_weights[token_idx, top_k_pos, None]
            final_hidden_states.index_add_(0, token_idx, current_hidden.to(final_hidden_states.dtype))
        return final_hidden_states.to(input_dtype)

    def _forward_decode(self, hidden_states, top_k_index, top_k_weights, compute_dtype, use_infer_gemv, input_dtype):
        """Single-token forward over the token's top-k experts with 0-d device indices, no host
        sync (``lora.py:409-460``)."""
        base = self.base
        final_hidden_states = torch.zeros_like(hidden_states, dtype=torch.float32)
        for j in range(top_k_index.shape[1]):
            expert_idx = top_k_index[0, j]
            proj = self._base_project(base.gate_up_proj, base.gate_up_absmax, base._gate_up_shape, expert_idx,
                                      hidden_states, compute_dtype, use_infer_gemv) + self._lora(
                hidden_states, self.gate_up_lora_A[expert_idx], self.gate_up_lora_B[expert_idx])
            current_hidden = _epilogue(base, proj)
            current_hidden = self._base_project(base.down_proj, base.down_absmax, base._down_shape, expert_idx,
                                                current_hidden, compute_dtype, use_infer_gemv) + self._lora(
                current_hidden, self.down_lora_A[expert_idx], self.down_lora_B[expert_idx])
            final_hidden_states += (current_hidden * top_k_weights[0, j]).to(final_hidden_states.dtype)
        return final_hidden_states.to(input_dtype)
