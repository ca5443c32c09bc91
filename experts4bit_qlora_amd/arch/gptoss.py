"""gpt-oss experts: per-expert biases + clamped GLU, over NF4 or MXFP4 storage.

``GptOssExperts4bit`` / ``GptOssExpertsNbit`` keep the reference classes
(``experts4bit_qlora/arch/gptoss.py:37-122``): dense weights de-interleaved at load (gate rows
``0::2`` then up rows ``1::2``, ``gptoss.py:66-68``), NF4 storage, forward
``(clamp(up)+1) * (g * sigmoid(alpha*g))`` with ``g = min(gate, limit)`` and both biases. The
reference's ``enable_fast`` SKIPS them (custom forward, biases), and so does this one.

``GptOssExpertsMxfp4`` is the MXFP4-resident form: the released e2m1/e8m0 bytes, rows
de-interleaved by a lossless row permutation, biases in the compute dtype. Its forward is the
same reference math with an MXFP4 dequant; ``enable_fast`` fuses it (MXFP4 decode in the GEMM,
bias + clamped GLU in the gate_up epilogue, bias in the down epilogue) -- the grouped form the
reference runs at ``engines/hot_residency.py:72-80`` over ``nvme_experts.py:852-865``'s MXFP4 kernel.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import quant as Q
from ..experts import Experts4bit, ExpertsNbit


class _GptOssForwardMixin:
    @classmethod
    def from_gptoss(cls, gate_up_dense, gate_up_bias, down_dense, down_bias, *, alpha: float = 1.702,
                    limit: float = 7.0, quant_type: str = "nf4", compute_dtype: torch.dtype = torch.bfloat16):
        """``gate_up_dense [E, hidden, 2*inter]`` (input-major, interleaved), ``gate_up_bias [E, 2*inter]``,
        ``down_dense [E, inter, hidden]``, ``down_bias [E, hidden]``."""
        if gate_up_dense.ndim != 3 or down_dense.ndim != 3:
            raise ValueError("expected [E, *, *] dense stacks")
        E, H, twoI = gate_up_dense.shape
        if twoI % 2:
            raise ValueError(f"gate_up last dim {twoI} not even")
        gu = gate_up_dense.transpose(1, 2).contiguous()
        gu = torch.cat([gu[:, 0::2, :], gu[:, 1::2, :]], dim=1)
        gub = torch.cat([gate_up_bias[:, 0::2], gate_up_bias[:, 1::2]], dim=1)
        dn = down_dense.transpose(1, 2).contiguous()
        base_cls = Experts4bit if quant_type in ("nf4", "fp4") else ExpertsNbit
        obj = base_cls.from_float(gu, dn, has_gate=True, quant_type=quant_type, compute_dtype=compute_dtype)
        obj.__class__ = GptOssExperts4bit if base_cls is Experts4bit else GptOssExpertsNbit
        obj.register_buffer("gate_up_bias", gub.to(compute_dtype), persistent=True)
        obj.register_buffer("down_bias", down_bias.to(compute_dtype), persistent=True)
        obj.alpha = float(alpha)
        obj.limit = float(limit)
        return obj

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
            gate_up = self._project(self.gate_up_proj, self.gate_up_absmax, self._gate_up_shape, e, x[tok], cd) \
                + self.gate_up_bias[e]
            gate, up = gate_up.chunk(2, dim=-1)
            gate = gate.clamp(max=self.limit)
            up = up.clamp(min=-self.limit, max=self.limit)
            gated = (up + 1) * (gate * torch.sigmoid(gate * self.alpha))
            h = self._project(self.down_proj, self.down_absmax, self._down_shape, e, gated, cd) + self.down_bias[e]
            h = h * router_scores[tok, pos, None]
            out.index_add_(0, tok, h.to(out.dtype))
        return out.to(input_dtype)


class GptOssExpertsNbit(_GptOssForwardMixin, ExpertsNbit):
    """gpt-oss experts over the general N-bit storage base."""


class GptOssExperts4bit(_GptOssForwardMixin, Experts4bit):
    """gpt-oss experts over the NF4/FP4 base."""


class GptOssExpertsMxfp4(nn.Module):
    """gpt-oss experts resident in MXFP4 with per-expert biases.

    Buffers (uint8 bytes exactly as released, rows de-interleaved to gate-block-then-up-block):
    ``gate_up_proj [E, 2I*H/2]``, ``gate_up_absmax [E, 2I*H/32]`` (e8m0), ``down_proj [E, H*I/2]``,
    ``down_absmax [E, H*I/32]``, biases ``gate_up_bias [E, 2I]`` / ``down_bias [E, H]`` in the compute
    dtype. Each row is one output feature with its ``in`` values contiguous.
    """

    quant_type = "mxfp4"
    bits = 4
    blocksize = 32
    has_gate = True

    def __init__(self, num_experts: int, hidden_dim: int, intermediate_dim: int, *, alpha: float = 1.702,
                 limit: float = 7.0, compute_dtype: torch.dtype = torch.bfloat16, device=None):
        super().__init__()
        for name, d in (("hidden_dim", hidden_dim), ("intermediate_dim", intermediate_dim)):
            if d % 32:
                raise ValueError(f"{name} ({d}) must be divisible by the MX block (32)")
        E, H, I = num_experts, hidden_dim, intermediate_dim
        self.num_experts, self.hidden_dim, self.intermediate_dim = E, H, I
        self.alpha, self.limit = float(alpha), float(limit)
        self.compute_dtype = compute_dtype
        self._gate_up_shape = (2 * I, H)
        self._down_shape = (H, I)
        u8 = dict(dtype=torch.uint8, device=device)
        self.gate_up_proj = nn.Parameter(torch.empty(E, 2 * I * H // 2, **u8), requires_grad=False)
        self.down_proj = nn.Parameter(torch.empty(E, H * I // 2, **u8), requires_grad=False)
        self.register_buffer("gate_up_absmax", torch.empty(E, 2 * I * H // 32, **u8))
        self.register_buffer("down_absmax", torch.empty(E, H * I // 32, **u8))
        self.register_buffer("gate_up_bias", torch.zeros(E, 2 * I, dtype=compute_dtype, device=device))
        self.register_buffer("down_bias", torch.zeros(E, H, dtype=compute_dtype, device=device))

    @classmethod
    def from_float(cls, gate_up: torch.Tensor, gate_up_bias: torch.Tensor, down: torch.Tensor,
                   down_bias: torch.Tensor, *, alpha: float = 1.702, limit: float = 7.0,
                   compute_dtype: torch.dtype = torch.bfloat16) -> "GptOssExpertsMxfp4":
        """Quantize e4b-layout stacks: ``gate_up [E, 2I, H]`` (gate block then up block),
        ``down [E, H, I]``; biases ``[E, 2I]`` and ``[E, H]`` in the same row order."""
        E, twoI, H = gate_up.shape
        I = twoI // 2
        if tuple(down.shape) != (E, H, I):
            raise ValueError(f"down {tuple(down.shape)} does not match gate_up {tuple(gate_up.shape)}")
        mod = cls(E, H, I, alpha=alpha, limit=limit, compute_dtype=compute_dtype, device=gate_up.device)
        gb, gs = Q.quantize_mxfp4(gate_up)
        db, ds = Q.quantize_mxfp4(down)
        mod.gate_up_proj.data = gb.reshape(E, -1).contiguous()
        mod.gate_up_absmax = gs.reshape(E, -1).contiguous()
        mod.down_proj.data = db.reshape(E, -1).contiguous()
        mod.down_absmax = ds.reshape(E, -1).contiguous()
        mod.gate_up_bias = gate_up_bias.to(compute_dtype).contiguous()
        mod.down_bias = down_bias.to(compute_dtype).contiguous()
        return mod

    @classmethod
    def from_gptoss_mxfp4(cls, gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales, down_bias,
                          *, alpha: float = 1.702, limit: float = 7.0,
                          compute_dtype: torch.dtype = torch.bfloat16) -> "GptOssExpertsMxfp4":
        """From the released tensors: ``gate_up_blocks [E, 2I, H/32, 16]`` / ``scales [E, 2I, H/32]`` with
        interleaved gate/up rows, ``down_blocks [E, H, I/32, 16]`` / ``scales [E, H, I/32]``, biases
        ``[E, 2I]`` (interleaved) and ``[E, H]``. The de-interleave (``gptoss.py:66-68``) is a row
        permutation of whole blocks and scales, so the bytes are kept exactly."""
        def u8(t):
            return t if t.dtype == torch.uint8 else t.view(torch.uint8)

        gb, gs, db, ds = u8(gate_up_blocks), u8(gate_up_scales), u8(down_blocks), u8(down_scales)
        E, twoI, G1, B = gb.shape
        H = G1 * B * 2
        I = twoI // 2
        if B != 16 or tuple(db.shape[:2]) != (E, H) or db.shape[2] * 32 != I:
            raise ValueError("unexpected gpt-oss MXFP4 shapes")
        perm = torch.cat([torch.arange(0, twoI, 2), torch.arange(1, twoI, 2)]).to(gb.device)
        mod = cls(E, H, I, alpha=alpha, limit=limit, compute_dtype=compute_dtype, device=gb.device)
        mod.gate_up_proj.data = gb.index_select(1, perm).reshape(E, -1).contiguous()
        mod.gate_up_absmax = gs.index_select(1, perm).reshape(E, -1).contiguous()
        mod.down_proj.data = db.reshape(E, -1).contiguous()
        mod.down_absmax = ds.reshape(E, -1).contiguous()
        mod.gate_up_bias = gate_up_bias.index_select(1, perm.to(gate_up_bias.device)).to(compute_dtype).contiguous()
        mod.down_bias = down_bias.to(compute_dtype).contiguous()
        return mod

    def _dequantize_expert(self, which: str, expert_idx, dtype: torch.dtype) -> torch.Tensor:
        """Dense ``[out, in]`` weight of one expert (bit-exact MXFP4 decode)."""
        packed = getattr(self, f"{which}_proj")[expert_idx]
        scales = getattr(self, f"{which}_absmax")[expert_idx]
        n, k = self._gate_up_shape if which == "gate_up" else self._down_shape
        if packed.is_cuda:
            from .. import ops

            qw = ops.mxfp4_qweight(packed.reshape(1, -1), scales.reshape(1, -1), n, k, num_experts=1)
            return ops.dequant(qw, 0, 1, dtype=dtype)[0]
        return Q.dequant_mxfp4_torch(packed, scales, n, k, dtype)

    def forward(self, hidden_states, router_indices, router_scores):
        """Reference math (``gptoss.py:83-114``) per hit expert over the MXFP4-decoded weights."""
        input_dtype = hidden_states.dtype
        cd = self.compute_dtype if self.compute_dtype is not None else input_dtype
        x = hidden_states.to(cd)
        out = torch.zeros_like(x, dtype=torch.float32)
        with torch.no_grad():
            mask = F.one_hot(router_indices, num_classes=self.num_experts).permute(2, 1, 0)
            hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero(as_tuple=False).view(-1)
        for e in hit:
            pos, tok = torch.where(mask[e])
            gate_up = F.linear(x[tok], self._dequantize_expert("gate_up", e, cd)) + self.gate_up_bias[e]
            gate, up = gate_up.chunk(2, dim=-1)
            gate = gate.clamp(max=self.limit)
            up = up.clamp(min=-self.limit, max=self.limit)
            gated = (up + 1) * (gate * torch.sigmoid(gate * self.alpha))
            h = F.linear(gated, self._dequantize_expert("down", e, cd)) + self.down_bias[e]
            h = h * router_scores[tok, pos, None]
            out.index_add_(0, tok, h.to(out.dtype))
        return out.to(input_dtype)
