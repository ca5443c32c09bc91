"""DeepSeek-V4 experts: clamped SwiGLU over NF4 storage (``experts4bit_qlora/arch/deepseek_v4.py``).

Only the expert math the fused path must reproduce is kept: ``_apply_gate`` (the hook
``lora._epilogue`` calls, ``deepseek_v4.py:178-195``: ``silu(min(gate, L)) * clamp(up, -L, L)`` in
fp32, ``L <= 0`` disables clamping) and the reference forward (``:197-225``: router weight applied
to the gated activation, in fp32, BEFORE the down projection). Checkpoint key maps are out of
scope. ``enable_fast`` fuses this epilogue into the gate_up kernel (``E4B_EPI_CLAMP_SWIGLU``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from ..experts import Experts4bit, ExpertsNbit

DEFAULT_SWIGLU_LIMIT = 10.0


class _DeepseekV4ForwardMixin:
    @classmethod
    def from_deepseek_v4(cls, gate_up_dense: torch.Tensor, down_dense: torch.Tensor, *,
                         limit: float = DEFAULT_SWIGLU_LIMIT, quant_type: str = "nf4",
                         compute_dtype: torch.dtype = torch.bfloat16, compress_statistics: bool = False):
        """``gate_up_dense [E, 2*inter, hidden]`` (``cat([w1, w3])``), ``down_dense [E, hidden, inter]``."""
        if gate_up_dense.ndim != 3 or down_dense.ndim != 3:
            raise ValueError("expected [E, *, *] dense stacks")
        E, twoI, H = gate_up_dense.shape
        if twoI % 2:
            raise ValueError(f"gate_up dim 1 = {twoI} is not even; cannot split gate/up")
        if tuple(down_dense.shape) != (E, H, twoI // 2):
            raise ValueError(f"down {tuple(down_dense.shape)} does not match gate_up {tuple(gate_up_dense.shape)}; "
                             f"expected {(E, H, twoI // 2)}")
        base_cls = Experts4bit if quant_type in ("nf4", "fp4") else ExpertsNbit
        obj = base_cls.from_float(gate_up_dense, down_dense, has_gate=True, quant_type=quant_type,
                                  compute_dtype=compute_dtype, compress_statistics=compress_statistics)
        obj.__class__ = DeepseekV4Experts4bit if base_cls is Experts4bit else DeepseekV4ExpertsNbit
        obj.limit = float(limit)
        return obj

    def _apply_gate(self, gate_up: torch.Tensor) -> torch.Tensor:
        """Clamped SwiGLU over a clean-concat gate_up, returned in fp32."""
        gate, up = gate_up.chunk(2, dim=-1)
        gate, up = gate.float(), up.float()
        if self.limit > 0:
            gate = gate.clamp(max=self.limit)
            up = up.clamp(min=-self.limit, max=self.limit)
        return F.silu(gate) * up

    def forward(self, hidden_states, router_indices, router_scores):
        input_dtype = hidden_states.dtype
        cd = self.compute_dtype if self.compute_dtype is not None else input_dtype
        x = hidden_states.to(cd)
        out = torch.zeros_like(x, dtype=torch.float32)
        with torch.no_grad():
            mask = F.one_hot(router_indices, num_classes=self.num_experts).permute(2, 1, 0)
            hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero(as_tuple=False).view(-1)
        for e in hit:
            pos, tok = torch.where(mask[e])
            gate_up = self._project(self.gate_up_proj, self.gate_up_absmax, self._gate_up_shape, e, x[tok], cd)
            gated = self._apply_gate(gate_up)
            gated = gated * router_scores[tok, pos, None].float()
            h = self._project(self.down_proj, self.down_absmax, self._down_shape, e, gated.to(cd), cd)
            out.index_add_(0, tok, h.to(out.dtype))
        return out.to(input_dtype)


class DeepseekV4ExpertsNbit(_DeepseekV4ForwardMixin, ExpertsNbit):
    """V4 experts over the general N-bit storage base."""


class DeepseekV4Experts4bit(_DeepseekV4ForwardMixin, Experts4bit):
    """V4 experts over the NF4/FP4 base (the fused path)."""
