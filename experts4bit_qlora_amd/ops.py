"""torch-tensor wrappers over the C ABI (``include/e4b_amd.h``).

Tensors are handed to the library as raw device pointers, the stream is torch's current HIP
stream, and every output / workspace is allocated by torch's caching allocator. No function
here synchronises the device, and none computes anything itself: a missing library raises
(:class:`experts4bit_qlora_amd._native.NativeUnavailable`).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _native as N

_DT = {torch.bfloat16: N.BF16, torch.float16: N.FP16, torch.float32: N.FP32}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    """The raw handle of torch's current stream on ``device`` (a CUDA device with its index):
    the accessor torch's own kernel launchers use, ~0.3 us against ~4 us for
    ``torch.cuda.current_stream(device).cuda_stream``, which an eager decode call pays each time."""
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None else torch.cuda.current_device())


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("the MI355X kernels need tensors on the HIP device")


@dataclass
class QW:
    """A 4-bit weight stack as the kernels see it (tensors kept alive alongside the struct)."""

    fmt: int
    num_experts: int
    n: int
    k: int
    packed: torch.Tensor
    absmax: torch.Tensor
    absmax2: torch.Tensor | None = None
    offset: torch.Tensor | None = None
    code: torch.Tensor | None = None
    code2: torch.Tensor | None = None
    bias: torch.Tensor | None = None
    shift: torch.Tensor | None = None  # NF4: per-expert exponents of the fp16 matrix-core mode

    def __setattr__(self, name, value):  # a changed field invalidates the cached descriptor
        self.__dict__.pop("_struct", None)
        self.__dict__.pop("_ref", None)
        object.__setattr__(self, name, value)

    def struct(self) -> N.QWeight:
        """The C descriptor, built once per field state: the tensors it points at are held by this
        object, and assigning any field drops it."""
        cached = self.__dict__.get("_struct")
        if cached is not None:
            return cached
        s = N.QWeight()
        s.format = self.fmt
        s.num_experts = self.num_experts
        s.n = self.n
        s.k = self.k
        s.packed = _ptr(self.packed)
        s.absmax = _ptr(self.absmax)
        s.absmax2 = _ptr(self.absmax2)
        s.offset = _ptr(self.offset)
        s.code = _ptr(self.code)
        s.code2 = _ptr(self.code2)
        s.bias = _ptr(self.bias)
        s.shift = _ptr(self.shift)
        self.__dict__["_struct"] = s
        self.__dict__["_ref"] = ctypes.byref(s)
        return s

    def ref(self):
        """``ctypes.byref(self.struct())``, kept with the descriptor (one less object per call)."""
        ref = self.__dict__.get("_ref")
        if ref is None:
            self.struct()
            ref = self.__dict__["_ref"]
        return ref


def with_weight_shift(qw: QW) -> QW:
    """Attach the per-expert exponents (``e4b_weight_shift``) that let the fused forward run its
    matrix-core GEMMs on fp16 operands; computed on the device, no synchronisation. A no-op for
    MXFP4 (exact in bf16) and for weights off the device."""
    if qw.fmt == N.FMT_MXFP4 or not qw.packed.is_cuda:
        return qw
    shift = torch.empty(qw.num_experts, dtype=torch.int32, device=qw.packed.device)
    s = qw.struct()
    N.check("e4b_weight_shift", N.lib().e4b_weight_shift(ctypes.byref(s), shift.data_ptr(), _stream(shift.device)))
    qw.shift = shift
    return qw


def nf4_qweight(packed, absmax, code, n, k, num_experts=None, bias=None) -> QW:
    """NF4 stack: ``packed`` u8 (any shape, ``E*n*k/2`` bytes), ``absmax`` fp32 ``E*n*k/64``."""
    E = num_experts if num_experts is not None else packed.shape[0]
    return QW(N.FMT_NF4, E, n, k, packed.contiguous(), absmax.contiguous().float(), code=code.contiguous().float(),
              bias=None if bias is None else bias.contiguous())


def nf4_dq_qweight(packed, qabsmax, absmax2, offset, code, code2, n, k, num_experts=None, bias=None) -> QW:
    E = num_experts if num_experts is not None else packed.shape[0]
    return QW(N.FMT_NF4_DQ, E, n, k, packed.contiguous(), qabsmax.contiguous(), absmax2.contiguous().float(),
              offset.contiguous().float(), code.contiguous().float(), code2.contiguous().float(),
              None if bias is None else bias.contiguous())


def mxfp4_qweight(blocks, scales, n, k, num_experts=None, bias=None) -> QW:
    E = num_experts if num_experts is not None else blocks.shape[0]

    def u8(t):
        return t if t.dtype == torch.uint8 else t.view(torch.uint8)

    return QW(N.FMT_MXFP4, E, n, k, u8(blocks).contiguous(), u8(scales).contiguous(),
              bias=None if bias is None else bias.contiguous())


# ------------------------------------------------------------------------------ dequant


def dequant(qw: QW, expert_begin: int = 0, expert_count: int | None = None, dtype=torch.float32) -> torch.Tensor:
    """Bit-exact dense ``[count, n, k]`` decode of experts ``[begin, begin+count)``."""
    _require_cuda(qw.packed)
    L = N.lib()
    count = qw.num_experts - expert_begin if expert_count is None else expert_count
    out = torch.empty(count, qw.n, qw.k, dtype=dtype, device=qw.packed.device)
    s = qw.struct()
    N.check("e4b_dequant", L.e4b_dequant(ctypes.byref(s), expert_begin, count, dtype_code(dtype), out.data_ptr(),
                                         _stream(out.device)))
    return out


# ------------------------------------------------------------------------------ routing


@dataclass
class RoutingBuffers:
    """Device routing (``e4b_routing``) for ``M = tokens * top_k`` rows."""

    sorted_flat: torch.Tensor
    inv: torch.Tensor
    offsets: torch.Tensor
    active: torch.Tensor
    tiles: torch.Tensor
    meta: torch.Tensor
    max_tiles: int
    tile_m: int
    scratch: torch.Tensor | None = None

    def struct(self) -> N.Routing:
        r = N.Routing()
        r.sorted_flat = self.sorted_flat.data_ptr()
        r.inv = self.inv.data_ptr()
        r.offsets = self.offsets.data_ptr()
        r.active = self.active.data_ptr()
        r.tiles = self.tiles.data_ptr()
        r.meta = self.meta.data_ptr()
        r.max_tiles = self.max_tiles
        r.tile_m = self.tile_m
        r.scratch = self.scratch.data_ptr() if self.scratch is not None else None
        return r


_TILE_M: list[int] = []


def mfma_tile_m() -> int:
    """Rows per MFMA tile of the library (a constant of the build; queried once)."""
    if not _TILE_M:
        _TILE_M.append(int(N.lib().e4b_mfma_tile_m()))
    return _TILE_M[0]


def route(top_k_index: torch.Tensor, num_experts: int, tile_m: int | None = None) -> RoutingBuffers:
    """Stable token->expert permutation on the device (no host sync)."""
    _require_cuda(top_k_index)
    L = N.lib()
    idx = top_k_index.to(torch.int64).contiguous()
    T, k = idx.shape
    M = T * k
    tm = tile_m or mfma_tile_m()
    max_tiles = max(1, -(-M // tm) + min(num_experts, M))
    dev = idx.device
    i32 = dict(dtype=torch.int32, device=dev)
    rb = RoutingBuffers(
        sorted_flat=torch.empty(max(M, 1), **i32),
        inv=torch.empty(max(M, 1), **i32),
        offsets=torch.empty(num_experts + 1, **i32),
        active=torch.empty(num_experts, **i32),
        tiles=torch.empty(2 * max_tiles, **i32),
        meta=torch.empty(4, **i32),
        max_tiles=max_tiles,
        tile_m=tm,
    )
    n_scratch = int(L.e4b_route_scratch_ints(M, num_experts))
    if n_scratch > 0:
        rb.scratch = torch.empty(n_scratch, **i32)
    rs = rb.struct()
    N.check("e4b_route", L.e4b_route(idx.data_ptr(), T, k, num_experts, ctypes.byref(rs), _stream(dev)))
    return rb


# -------------------------------------------------------------------------------- GEMMs


def grouped_gemm(a: torch.Tensor, qw: QW, rb: RoutingBuffers, tokens: int, M: int, epilogue: int = N.EPI_NONE,
                 gather_k: int = 0, alpha: float = 1.702, limit: float = 7.0, path: int = N.PATH_AUTO,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Grouped GEMM over expert-sorted rows with an optional fused epilogue; ``[M, n_out]`` in
    ``out_dtype`` (default: ``a``'s dtype; ``torch.float32`` keeps the fp32 result)."""
    _require_cuda(a, qw.packed)
    L = N.lib()
    a = a.contiguous()
    gated = epilogue in (N.EPI_SWIGLU, N.EPI_CLAMP_SWIGLU, N.EPI_GPTOSS)
    n_out = qw.n // 2 if gated else qw.n
    od = a.dtype if out_dtype is None else out_dtype
    out = torch.empty(M, n_out, dtype=od, device=a.device)
    s = qw.struct()
    rs = rb.struct()
    N.check("e4b_grouped_gemm",
            L.e4b_grouped_gemm(a.data_ptr(), dtype_code(a.dtype), gather_k, ctypes.byref(s), ctypes.byref(rs),
                               tokens, M, epilogue, float(alpha), float(limit), path, out.data_ptr(), dtype_code(od),
                               _stream(a.device)))
    return out


def combine(down: torch.Tensor, rb: RoutingBuffers, top_k_weights: torch.Tensor, tokens: int, top_k: int,
            out_dtype: torch.dtype) -> torch.Tensor:
    """Deterministic weighted k-sum back to token order (``[tokens, hidden]`` in ``out_dtype``)."""
    _require_cuda(down, top_k_weights)
    L = N.lib()
    H = down.shape[1]
    w = top_k_weights.contiguous()
    out = torch.empty(tokens, H, dtype=out_dtype, device=down.device)
    N.check("e4b_combine",
            L.e4b_combine(down.data_ptr(), dtype_code(down.dtype), rb.inv.data_ptr(), w.data_ptr(),
                          dtype_code(w.dtype), tokens, top_k, H, out.data_ptr(), dtype_code(out_dtype),
                          _stream(down.device)))
    return out


def lora_delta(x: torch.Tensor, rb: RoutingBuffers, M: int, num_experts: int, lora_a: torch.Tensor,
               lora_b: torch.Tensor, scaling: float, out: torch.Tensor, gather_k: int = 0,
               delta_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Add the per-expert low-rank delta to ``out`` (``[M, out_features]`` fp32, expert-sorted
    rows) in place: ``out[m] += delta_dtype(scaling * (x_m @ A[e].T) @ B[e].T)`` for every routed
    row, all groups in one pass (``lora.py:251-256`` per group as ``fast.py:229-233`` applies it,
    without the host's group sizes). ``x_m`` is ``x[sorted_flat[m] // gather_k]`` when
    ``gather_k > 0`` (token rows), else ``x[m]``; ``delta_dtype`` defaults to ``x.dtype``."""
    _require_cuda(x, lora_a, lora_b, out)
    if out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp32 tensor")
    L = N.lib()
    xc = x.contiguous()
    a = lora_a.contiguous()
    b = lora_b.to(a.dtype).contiguous()
    E, r, k_in = a.shape
    n_out = b.shape[1]
    t = torch.empty(max(M, 1), r, dtype=torch.float32, device=x.device)
    rt = rb.struct()
    N.check("e4b_lora_delta",
            L.e4b_lora_delta(xc.data_ptr(), dtype_code(xc.dtype), gather_k, ctypes.byref(rt), M, num_experts,
                             a.data_ptr(), b.data_ptr(), dtype_code(a.dtype), r, k_in, n_out, float(scaling),
                             dtype_code(delta_dtype or xc.dtype), t.data_ptr(), out.data_ptr(), _stream(x.device)))
    return out


def lora_t(x: torch.Tensor, rb: RoutingBuffers, M: int, num_experts: int, lora_a: torch.Tensor,
           gather_k: int = 0) -> torch.Tensor:
    """``t[m] = x_m @ A[e_m].T`` for the expert-sorted rows: fp32 ``[M, r]`` (``lora_a [E, r, in]``
    in any dtype; ``x_m`` as for :func:`lora_delta`). Rows past the routed ones are left unset."""
    _require_cuda(x, lora_a)
    L = N.lib()
    xc = x.contiguous()
    a = lora_a.contiguous()
    E, r, k_in = a.shape
    t = torch.empty(max(M, 1), r, dtype=torch.float32, device=x.device)
    rt = rb.struct()
    N.check("e4b_lora_t",
            L.e4b_lora_t(xc.data_ptr(), dtype_code(xc.dtype), gather_k, ctypes.byref(rt), M, num_experts, a.data_ptr(),
                         dtype_code(a.dtype), r, k_in, t.data_ptr(), _stream(x.device)))
    return t[:M]


def lora_t_add(t: torch.Tensor, rb: RoutingBuffers, M: int, num_experts: int, lora_b: torch.Tensor, scaling: float,
               out: torch.Tensor, delta_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``out[m] += delta_dtype(scaling * t[m] @ B[e_m].T)`` in place for the routed rows (``t`` fp32
    ``[M, r]``, ``lora_b [E, out_features, r]``, ``out`` fp32 ``[M, out_features]``)."""
    _require_cuda(t, lora_b, out)
    if out.dtype != torch.float32 or not out.is_contiguous() or t.dtype != torch.float32:
        raise ValueError("t and out must be fp32, out contiguous")
    L = N.lib()
    tc = t.contiguous()
    b = lora_b.contiguous()
    E, n_out, r = b.shape
    rt = rb.struct()
    N.check("e4b_lora_t_add",
            L.e4b_lora_t_add(tc.data_ptr(), ctypes.byref(rt), M, num_experts, b.data_ptr(), dtype_code(b.dtype), r,
                             n_out, float(scaling), dtype_code(delta_dtype), out.data_ptr(), _stream(t.device)))
    return out


def lora_wgrad(u: torch.Tensor, a: torch.Tensor, rb: RoutingBuffers, M: int, num_experts: int, scale: float,
               gather_k: int = 0) -> torch.Tensor:
    """Per-expert ``out[e] = scale * u_e.T @ a_e`` over expert e's sorted rows: fp32 ``[E, r, cols]``
    (``u`` fp32 ``[M, r]``; ``a_m`` = ``a[sorted_flat[m] // gather_k]`` or ``a[m]``)."""
    _require_cuda(u, a)
    L = N.lib()
    uc = u.contiguous()
    ac = a.contiguous()
    r = uc.shape[1]
    cols = ac.shape[1]
    out = torch.empty(num_experts, r, cols, dtype=torch.float32, device=a.device)
    rt = rb.struct()
    N.check("e4b_lora_wgrad",
            L.e4b_lora_wgrad(uc.data_ptr(), r, ac.data_ptr(), dtype_code(ac.dtype), gather_k, ctypes.byref(rt), M,
                             num_experts, cols, float(scale), out.data_ptr(), _stream(a.device)))
    return out


def grouped_dgrad(g: torch.Tensor, qw: QW, rb: RoutingBuffers, M: int) -> torch.Tensor:
    """Input gradient of a frozen grouped projection: ``out[m] = g[m] @ deq(W[e_m])`` over the
    expert-sorted rows, fp32 ``[M, k]`` (``g [M, n]`` bf16 / fp16; ``rb.tile_m`` 128 or 32)."""
    _require_cuda(g, qw.packed)
    L = N.lib()
    gc = g.contiguous()
    out = torch.empty(max(M, 1), qw.k, dtype=torch.float32, device=g.device)
    s = qw.struct()
    rt = rb.struct()
    N.check("e4b_grouped_dgrad",
            L.e4b_grouped_dgrad(gc.data_ptr(), dtype_code(gc.dtype), ctypes.byref(s), ctypes.byref(rt), M,
                                out.data_ptr(), _stream(g.device)))
    return out[:M]


def lora_delta_epilogue(x: torch.Tensor, rb: RoutingBuffers, M: int, num_experts: int, lora_a: torch.Tensor,
                        lora_b: torch.Tensor, scaling: float, proj: torch.Tensor, epilogue: int, limit: float = 0.0,
                        gather_k: int = 0, h_dtype: torch.dtype | None = None,
                        delta_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The gate_up projection's LoRA delta fused with the activation: returns ``h`` ``[M, n']``
    (``n' = out_features / 2`` for ``EPI_SWIGLU`` / ``EPI_CLAMP_SWIGLU``, else ``out_features``)
    in ``h_dtype`` (default ``x.dtype``), ``h[m] = epilogue(proj[m] + delta_dtype(scaling * (x_m @
    A[e].T) @ B[e].T))`` for every routed row (``delta_dtype``: ``h_dtype`` by default, as the
    reference's ``_lora`` casts it back, or ``torch.float32`` to leave it unrounded); ``proj``
    (fp32, expert-sorted rows) is not written. Rows past the routed ones are left unset."""
    _require_cuda(x, lora_a, lora_b, proj)
    if proj.dtype != torch.float32 or not proj.is_contiguous():
        raise ValueError("proj must be a contiguous fp32 tensor")
    L = N.lib()
    xc = x.contiguous()
    a = lora_a.contiguous()
    b = lora_b.to(a.dtype).contiguous()
    E, r, k_in = a.shape
    n_out = b.shape[1]
    gated = epilogue in (N.EPI_SWIGLU, N.EPI_CLAMP_SWIGLU)
    hd = h_dtype or xc.dtype
    h = torch.empty(M, n_out // 2 if gated else n_out, dtype=hd, device=x.device)
    t = torch.empty(max(M, 1), r, dtype=torch.float32, device=x.device)
    rt = rb.struct()
    N.check("e4b_lora_delta_epilogue",
            L.e4b_lora_delta_epilogue(xc.data_ptr(), dtype_code(xc.dtype), gather_k, ctypes.byref(rt), M, num_experts,
                                      a.data_ptr(), b.data_ptr(), dtype_code(a.dtype), r, k_in, n_out, float(scaling),
                                      dtype_code(delta_dtype or hd), t.data_ptr(), proj.data_ptr(), int(epilogue),
                                      float(limit), h.data_ptr(), dtype_code(hd), _stream(x.device)))
    return h


def decode_gate_up(hidden: torch.Tensor, top_k_index: torch.Tensor, w1: QW, epilogue: int, alpha: float = 1.702,
                   limit: float = 7.0) -> torch.Tensor:
    """Decode-path gate_up (routing recomputed on the device): ``h [tokens * k, h_cols]`` in flat
    (token, slot) order."""
    _require_cuda(hidden, top_k_index, w1.packed)
    L = N.lib()
    x = hidden.contiguous()
    idx = top_k_index.to(torch.int64).contiguous()
    T, k = idx.shape
    gated = epilogue in (N.EPI_SWIGLU, N.EPI_CLAMP_SWIGLU, N.EPI_GPTOSS)
    h = torch.empty(T * k, w1.n // 2 if gated else w1.n, dtype=x.dtype, device=x.device)
    s1 = w1.struct()
    N.check("e4b_decode_gate_up",
            L.e4b_decode_gate_up(x.data_ptr(), dtype_code(x.dtype), T, idx.data_ptr(), k, ctypes.byref(s1), epilogue,
                                 float(alpha), float(limit), h.data_ptr(), _stream(x.device)))
    return h


def decode_down_combine(h: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor, w2: QW,
                        out_dtype: torch.dtype) -> torch.Tensor:
    """Decode-path down projection fused with the deterministic k-slot combine: ``[tokens, n]``."""
    _require_cuda(h, top_k_index, top_k_weights, w2.packed)
    L = N.lib()
    idx = top_k_index.to(torch.int64).contiguous()
    w = top_k_weights.contiguous()
    T, k = idx.shape
    out = torch.empty(T, w2.n, dtype=out_dtype, device=h.device)
    s2 = w2.struct()
    N.check("e4b_decode_down_combine",
            L.e4b_decode_down_combine(h.contiguous().data_ptr(), dtype_code(h.dtype), T, idx.data_ptr(), w.data_ptr(),
                                      dtype_code(w.dtype), k, ctypes.byref(s2), out.data_ptr(), dtype_code(out_dtype),
                                      _stream(h.device)))
    return out


# workspace sizes by (tokens, top_k, E, n1, n2, epilogue, act dtype): a pure function of its
# arguments, asked once per shape instead of once per call
_MOE_WS: dict = {}


def _moe_ws_bytes(*key) -> int:
    b = _MOE_WS.get(key)
    if b is None:
        if len(_MOE_WS) > 4096:
            _MOE_WS.clear()
        b = _MOE_WS[key] = int(N.lib().e4b_moe_workspace_bytes(*key))
    return b


def moe_forward(hidden: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor, w1: QW, w2: QW,
                epilogue: int, out_dtype: torch.dtype, alpha: float = 1.702, limit: float = 7.0,
                path: int = N.PATH_AUTO) -> torch.Tensor:
    """The whole fused expert forward in one C-ABI call (route, gate_up+epilogue, down, combine).
    Per call the host does only what the call needs (an eager decode layer is host-bound): the
    workspace size is memoised per shape and the descriptors' ``byref`` kept with them."""
    _require_cuda(hidden, top_k_index, top_k_weights, w1.packed, w2.packed)
    x = hidden.contiguous()
    idx = top_k_index if top_k_index.dtype == torch.int64 else top_k_index.to(torch.int64)
    idx = idx.contiguous()
    w = top_k_weights.contiguous()
    T, k = idx.shape
    adt = dtype_code(x.dtype)
    ws_bytes = _moe_ws_bytes(T, k, w1.num_experts, w1.n, w2.n, epilogue, adt)
    dev = x.device
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    out = torch.empty(T, w2.n, dtype=out_dtype, device=dev)
    N.check("e4b_moe_forward",
            N.lib().e4b_moe_forward(x.data_ptr(), adt, T, idx.data_ptr(), w.data_ptr(), dtype_code(w.dtype), k,
                                    w1.ref(), w2.ref(), epilogue, float(alpha), float(limit), path, ws.data_ptr(),
                                    ws_bytes, out.data_ptr(), dtype_code(out_dtype), _stream(dev)))
    return out


def moe_lora_forward(hidden: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor, w1: QW, w2: QW,
                     lora1: tuple[torch.Tensor, torch.Tensor], lora2: tuple[torch.Tensor, torch.Tensor],
                     scaling: float, epilogue: int, out_dtype: torch.dtype, limit: float = 7.0,
                     path: int = N.PATH_AUTO) -> torch.Tensor:
    """The fused ExpertsLoRA forward in one C-ABI call (``e4b_moe_lora_forward``): ``lora1 =
    (A1 [E, r, H], B1 [E, n1, r])`` of the gate_up projection, ``lora2 = (A2 [E, r, I],
    B2 [E, H, r])`` of the down projection, all in one dtype (B is converted to A's if not)."""
    _require_cuda(hidden, top_k_index, top_k_weights, w1.packed, w2.packed, *lora1, *lora2)
    L = N.lib()
    x = hidden.contiguous()
    idx = top_k_index.to(torch.int64).contiguous()
    w = top_k_weights.contiguous()
    T, k = idx.shape
    a1 = lora1[0].contiguous()
    adt = a1.dtype
    b1 = lora1[1].to(adt).contiguous()
    a2 = lora2[0].to(adt).contiguous()
    b2 = lora2[1].to(adt).contiguous()
    r = int(a1.shape[1])
    ws_bytes = int(L.e4b_moe_lora_workspace_bytes(T, k, w1.num_experts, w1.n, w2.n, epilogue, dtype_code(x.dtype), r))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty(T, w2.n, dtype=out_dtype, device=x.device)
    s1, s2 = w1.struct(), w2.struct()
    lo = N.Lora(a1=a1.data_ptr(), b1=b1.data_ptr(), a2=a2.data_ptr(), b2=b2.data_ptr(), dtype=dtype_code(adt), rank=r,
                scaling=float(scaling))
    N.check("e4b_moe_lora_forward",
            L.e4b_moe_lora_forward(x.data_ptr(), dtype_code(x.dtype), T, idx.data_ptr(), w.data_ptr(),
                                   dtype_code(w.dtype), k, ctypes.byref(s1), ctypes.byref(s2), ctypes.byref(lo),
                                   epilogue, float(limit), path, ws.data_ptr(), ws_bytes, out.data_ptr(),
                                   dtype_code(out_dtype), _stream(x.device)))
    return out


# ------------------------------------------------- the nf4_grouped / mxfp4_grouped API shape


def _routing_from_sizes(sizes, expert_ids, num_experts: int, device) -> tuple[RoutingBuffers, int]:
    """Host-described groups (the reference's ``sizes`` / ``expert_ids`` lists) -> device routing."""
    sizes = [int(s) for s in sizes]
    ids = [int(e) for e in (expert_ids.tolist() if torch.is_tensor(expert_ids) else expert_ids)]
    if len(sizes) != len(ids):
        raise ValueError("sizes and expert_ids differ in length")
    if any(s < 0 for s in sizes) or any(not 0 <= e < num_experts for e in ids):
        raise ValueError("bad group sizes / expert ids")
    if len(set(ids)) != len(ids) or ids != sorted(ids):
        raise ValueError("expert_ids must be strictly ascending (one group per expert)")
    M = sum(sizes)
    tm = mfma_tile_m()
    counts = [0] * num_experts
    for e, s in zip(ids, sizes):
        counts[e] = s
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    active = [e for e in range(num_experts) if counts[e] > 0]
    tiles = []
    for e in active:
        for t in range(-(-counts[e] // tm)):
            tiles += [e, offsets[e] + t * tm]
    max_tiles = max(1, len(tiles) // 2)
    i32 = dict(dtype=torch.int32, device=device)
    ar = torch.arange(max(M, 1), **i32)
    rb = RoutingBuffers(
        sorted_flat=ar, inv=ar,
        offsets=torch.tensor(offsets, **i32),
        active=torch.tensor(active + [0] * (num_experts - len(active)), **i32),
        tiles=torch.tensor(tiles or [0, 0], **i32),
        meta=torch.tensor([len(tiles) // 2, len(active), 0, tm], **i32),
        max_tiles=max_tiles, tile_m=tm,
    )
    return rb, M


def route_groups(sizes, expert_ids: torch.Tensor, num_experts: int, tile_m: int | None = None) -> RoutingBuffers:
    """Routing of row groups with host ``sizes`` and device ``expert_ids`` (``e4b_route_groups``):
    no host read-back of the ids, nothing copied between host and device."""
    _require_cuda(expert_ids)
    L = N.lib()
    ids = expert_ids.to(torch.int64).contiguous()
    G = len(sizes)
    if ids.numel() != G:
        raise ValueError("sizes and expert_ids differ in length")
    M = int(sum(int(s) for s in sizes))
    tm = tile_m or mfma_tile_m()
    max_tiles = max(1, -(-M // tm) + min(num_experts, G))
    i32 = dict(dtype=torch.int32, device=ids.device)
    rb = RoutingBuffers(
        sorted_flat=torch.empty(max(M, 1), **i32),
        inv=torch.empty(max(M, 1), **i32),
        offsets=torch.empty(num_experts + 1, **i32),
        active=torch.empty(num_experts, **i32),
        tiles=torch.empty(2 * max_tiles, **i32),
        meta=torch.empty(4, **i32),
        max_tiles=max_tiles,
        tile_m=tm,
    )
    host_sizes = (ctypes.c_int64 * max(G, 1))(*[int(s) for s in sizes])
    rs = rb.struct()
    N.check("e4b_route_groups", L.e4b_route_groups(host_sizes, G, ids.data_ptr(), num_experts, ctypes.byref(rs),
                                                   _stream(ids.device)))
    return rb


def _grouped_call(a: torch.Tensor, qw: QW, sizes, expert_ids) -> torch.Tensor:
    """The reference grouped call on ``qw``: host id lists route on the host side as before; a
    device id tensor routes on the device and the rows come back in group order through ``inv``
    (rows of an out-of-range id are zero), all without a synchronisation."""
    if torch.is_tensor(expert_ids) and expert_ids.is_cuda:
        M = int(sum(int(s) for s in sizes))
        if a.shape[0] != M:
            raise ValueError(f"a has {a.shape[0]} rows but sizes sum to {M}")
        rb = route_groups(sizes, expert_ids, qw.num_experts)
        tokens = max((int(s) for s in sizes), default=0)
        out = grouped_gemm(a, qw, rb, tokens, M, gather_k=1)
        inv = rb.inv[:M].long()
        return out.index_select(0, inv.clamp(min=0)).masked_fill_((inv < 0).unsqueeze(1), 0)
    rb, M = _routing_from_sizes(sizes, expert_ids, qw.num_experts, qw.packed.device)
    if a.shape[0] != M:
        raise ValueError(f"a has {a.shape[0]} rows but sizes sum to {M}")
    tokens = max(sizes) if len(sizes) else 0
    return grouped_gemm(a, qw, rb, tokens, M)


def gemm_4bit_grouped(a: torch.Tensor, w: torch.Tensor, absmax: torch.Tensor, sizes, expert_ids,
                      code: torch.Tensor | None = None) -> torch.Tensor:
    """Drop-in for ``nf4_grouped.gemm_4bit_grouped(a, w[E,N,K/2], absmax[E,N,K/64], sizes, ids)``
    (the call shapes at engines/fast.py:137-156 -- host ids -- and engines/pipelined.py:502-508 --
    device ids, no synchronisation): ``[M, N]`` in ``a``'s dtype."""
    E, n, kh = w.shape
    c = code if code is not None else _nf4_code_on(w.device)
    qw = nf4_qweight(w, absmax, c, n, kh * 2, num_experts=E)
    return _grouped_call(a, qw, sizes, expert_ids)


_NF4_CODE: dict = {}


def _nf4_code_on(device) -> torch.Tensor:
    """The NF4 code table on ``device``, made once (a host-to-device copy per call would
    synchronise)."""
    from .quant import code_4bit

    key = torch.device(device)
    t = _NF4_CODE.get(key)
    if t is None:
        t = _NF4_CODE[key] = code_4bit("nf4", device=key)
    return t


def gemm_mxfp4_grouped(a: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, sizes, expert_ids) -> torch.Tensor:
    """Drop-in for ``mxfp4_grouped.gemm_mxfp4_grouped(a, blocks[E,N,K/2], scales[E,N,K/32], sizes, ids)``
    (engines/nvme_experts.py:852-865); host or device ids as for gemm_4bit_grouped."""
    E, n, kh = blocks.shape
    qw = mxfp4_qweight(blocks, scales, n, kh * 2, num_experts=E)
    return _grouped_call(a, qw, sizes, expert_ids)


def gather_rows(dst: torch.Tensor, src_addr: torch.Tensor, ident: torch.Tensor, have: torch.Tensor, n_bytes: int,
                dst_off: int = 0, bytes_copied: torch.Tensor | None = None) -> None:
    """Address-table row gather (``e4b_gather_rows``): slot s of ``dst`` (``[slots, row]``, any
    dtype, contiguous) receives ``n_bytes`` read at the absolute address ``src_addr[s]`` at byte
    ``dst_off`` of its row, unless ``ident[s] == have[s]``. ``bytes_copied`` (a device int64 scalar)
    accumulates the bytes moved. Enqueued on the current stream; nothing is read back."""
    _require_cuda(dst, src_addr, ident, have)
    if not dst.is_contiguous() or dst.dim() < 2:
        raise ValueError("dst must be a contiguous [slots, row...] tensor")
    for t in (src_addr, ident, have):
        if t.dtype != torch.int64 or not t.is_contiguous() or t.numel() != dst.shape[0]:
            raise ValueError("src_addr, ident and have must be contiguous int64 with one entry per slot")
    row_bytes = dst[0].numel() * dst.element_size()
    cp = None
    if bytes_copied is not None:
        if bytes_copied.dtype != torch.int64 or not bytes_copied.is_cuda or bytes_copied.numel() != 1:
            raise ValueError("bytes_copied must be a one-element int64 device tensor")
        cp = bytes_copied.data_ptr()
    N.check("e4b_gather_rows",
            N.lib().e4b_gather_rows(dst.data_ptr(), row_bytes, int(dst_off), src_addr.data_ptr(), ident.data_ptr(),
                                    have.data_ptr(), dst.shape[0], int(n_bytes), cp, _stream(dst.device)))
