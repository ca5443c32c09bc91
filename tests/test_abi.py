"""The C-ABI library: it loads, exports every symbol ``include/e4b_amd.h`` declares, and its host
logic rejects bad arguments with a status and a message -- all without touching a GPU (every
call below returns before any HIP launch)."""
import ctypes
import os
import re

import pytest

from experts4bit_qlora_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "e4b_amd.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(e4b_[a-z_0-9]+)\s*\(", src)))


def test_library_is_built_and_loads():
    assert N.available(), N._load_error
    assert N.lib().e4b_version().startswith(b"e4b_amd")


def test_exports_every_declared_symbol():
    declared = _declared()
    assert declared, "no declarations parsed from the header"
    assert sorted(N.EXPORTS) == declared
    raw = ctypes.CDLL(N.LIB_PATH)
    for name in declared:
        assert hasattr(raw, name), f"{name} declared in include/e4b_amd.h but not exported"


def test_enums_match_header():
    src = open(HEADER).read()
    for name, val in (("E4B_FMT_NF4", N.FMT_NF4), ("E4B_FMT_NF4_DQ", N.FMT_NF4_DQ), ("E4B_FMT_MXFP4", N.FMT_MXFP4),
                      ("E4B_BF16", N.BF16), ("E4B_FP16", N.FP16), ("E4B_FP32", N.FP32),
                      ("E4B_EPI_NONE", N.EPI_NONE), ("E4B_EPI_SWIGLU", N.EPI_SWIGLU), ("E4B_EPI_ACT", N.EPI_ACT),
                      ("E4B_EPI_CLAMP_SWIGLU", N.EPI_CLAMP_SWIGLU), ("E4B_EPI_GPTOSS", N.EPI_GPTOSS),
                      ("E4B_PATH_AUTO", N.PATH_AUTO), ("E4B_PATH_GEMV", N.PATH_GEMV),
                      ("E4B_PATH_MFMA", N.PATH_MFMA)):
        m = re.search(rf"\b{name}\s*=\s*(-?\d+)", src)
        assert m and int(m.group(1)) == val, name


def test_struct_layouts():
    assert ctypes.sizeof(N.QWeight) == 4 + 4 + 8 + 8 + 8 * 8
    assert N.QWeight.shift.offset == 4 + 4 + 8 + 8 + 7 * 8  # the last field, after bias
    assert ctypes.sizeof(N.Routing) == 6 * 8 + 4 + 4 + 8


def test_weight_shift_rejects_bad_arguments():
    """Validation happens before any launch, so it runs without a device."""
    L = N.lib()
    s = _qw(format=N.FMT_MXFP4)
    assert L.e4b_weight_shift(ctypes.byref(s), 4096, None) == -2
    assert "MXFP4" in _err()
    s = _qw()
    assert L.e4b_weight_shift(ctypes.byref(s), None, None) == -1
    assert "NULL" in _err()


def _qw(**kw):
    s = N.QWeight()
    s.format, s.num_experts, s.n, s.k = kw.get("format", N.FMT_NF4), kw.get("E", 2), kw.get("n", 64), kw.get("k", 64)
    s.packed = kw.get("packed", 4096)
    s.absmax = kw.get("absmax", 8192)
    s.code = kw.get("code", 16384)
    return s


def _err():
    return N.lib().e4b_last_error().decode()


def test_dequant_rejects_bad_arguments():
    L = N.lib()
    assert L.e4b_dequant(None, 0, 1, N.FP32, 4096, None) == -1
    assert "NULL" in _err()
    s = _qw(k=96)
    assert L.e4b_dequant(ctypes.byref(s), 0, 1, N.FP32, 4096, None) == -2
    assert "multiple of 64" in _err()
    s = _qw()
    assert L.e4b_dequant(ctypes.byref(s), 1, 2, N.FP32, 4096, None) == -1
    assert "expert range" in _err()
    assert L.e4b_dequant(ctypes.byref(s), 0, 1, 7, 4096, None) == -1
    s = _qw(format=N.FMT_NF4_DQ)
    assert L.e4b_dequant(ctypes.byref(s), 0, 1, N.FP32, 4096, None) == -1
    assert "double-quant" in _err()
    s = _qw(packed=4097)
    assert L.e4b_dequant(ctypes.byref(s), 0, 1, N.FP32, 4096, None) == -1
    assert "aligned" in _err()
    # an empty range is a valid no-op
    s = _qw()
    assert L.e4b_dequant(ctypes.byref(s), 0, 0, N.FP32, 4096, None) == 0


def _rt(max_tiles=8, tile_m=64):
    r = N.Routing()
    r.sorted_flat = r.inv = r.offsets = r.active = r.tiles = r.meta = 4096
    r.max_tiles, r.tile_m = max_tiles, tile_m
    return r


def test_route_rejects_bad_arguments():
    L = N.lib()
    r = _rt()
    assert L.e4b_route(4096, 4, 2, 0, ctypes.byref(r), None) == -2
    assert L.e4b_route(4096, 4, 2, 4096, ctypes.byref(r), None) == -2
    assert L.e4b_route(4096, -1, 2, 8, ctypes.byref(r), None) == -1
    small = _rt(max_tiles=1)
    assert L.e4b_route(4096, 100, 8, 64, ctypes.byref(small), None) == -4
    assert "max_tiles" in _err()
    bad = _rt()
    bad.meta = None
    assert L.e4b_route(4096, 4, 2, 8, ctypes.byref(bad), None) == -1


def test_route_scratch_sizes():
    L = N.lib()
    assert L.e4b_route_scratch_ints(4096, 128) == 0  # one workgroup routes up to 4096 rows
    assert L.e4b_route_scratch_ints(4097, 128) == 17 * 129
    assert L.e4b_route_scratch_ints(32768, 128) == 128 * 129
    r = _rt(max_tiles=1000)
    assert L.e4b_route(4096, 8192, 1, 8, ctypes.byref(r), None) == -1  # 8192 rows, scratch NULL
    assert "scratch" in _err()


def test_grouped_gemm_rejects_bad_arguments():
    L = N.lib()
    s, r = _qw(n=63), _rt()
    assert L.e4b_grouped_gemm(4096, N.BF16, 0, ctypes.byref(s), ctypes.byref(r), 1, 2, N.EPI_SWIGLU, 1.0, 7.0, 0,
                              8192, N.BF16, None) == -1
    assert "even n" in _err()
    s = _qw()
    assert L.e4b_grouped_gemm(4096, N.FP32, 0, ctypes.byref(s), ctypes.byref(r), 1, 2, N.EPI_NONE, 1.0, 7.0, 0,
                              8192, N.FP32, None) == -1
    assert L.e4b_grouped_gemm(4096, N.BF16, 0, ctypes.byref(s), ctypes.byref(r), 1, 2, N.EPI_GPTOSS, 1.0, 7.0, 0,
                              8192, N.BF16, None) == -1
    assert "bias" in _err()
    r64 = _rt(tile_m=64)
    assert L.e4b_grouped_gemm(4096, N.BF16, 0, ctypes.byref(s), ctypes.byref(r64), 64, 128, N.EPI_NONE, 1.0, 7.0,
                              N.PATH_MFMA, 8192, N.BF16, None) == -1
    assert "tile_m" in _err()
    assert L.e4b_grouped_gemm(4096, N.BF16, 0, ctypes.byref(s), ctypes.byref(r), 1, 2, N.EPI_NONE, 1.0, 7.0, 0,
                              8192, N.FP16, None) == -1
    assert "out_dtype" in _err()
    # M == 0 is a valid no-op
    assert L.e4b_grouped_gemm(4096, N.BF16, 0, ctypes.byref(s), ctypes.byref(r), 0, 0, N.EPI_NONE, 1.0, 7.0, 0,
                              8192, N.BF16, None) == 0


def test_moe_forward_checks_shapes_and_workspace():
    L = N.lib()
    w1, w2 = _qw(n=128, k=64), _qw(n=64, k=128)  # gate_up out 128 -> h 64, but down k 128
    assert L.e4b_moe_forward(4096, N.BF16, 2, 4096, 4096, N.BF16, 2, ctypes.byref(w1), ctypes.byref(w2),
                             N.EPI_SWIGLU, 1.0, 7.0, 0, 4096, 1 << 20, 8192, N.BF16, None) == -1
    assert "does not match" in _err()
    w2 = _qw(n=64, k=64)
    need = L.e4b_moe_workspace_bytes(2, 2, 2, 128, 64, N.EPI_SWIGLU, N.BF16)
    assert need > 0
    assert L.e4b_moe_forward(4096, N.BF16, 2, 4096, 4096, N.BF16, 2, ctypes.byref(w1), ctypes.byref(w2),
                             N.EPI_SWIGLU, 1.0, 7.0, 0, 4096, need - 1, 8192, N.BF16, None) == -4
    assert "workspace" in _err()
    # tokens == 0 is a valid no-op
    assert L.e4b_moe_forward(4096, N.BF16, 0, 4096, 4096, N.BF16, 2, ctypes.byref(w1), ctypes.byref(w2),
                             N.EPI_SWIGLU, 1.0, 7.0, 0, 4096, 0, 8192, N.BF16, None) == 0


def _lora(rank=16, dtype=N.FP32, scaling=2.0):
    return N.Lora(a1=4096, b1=4096, a2=4096, b2=4096, dtype=dtype, rank=rank, scaling=scaling)


def test_lora_struct_layout():
    assert ctypes.sizeof(N.Lora) == 4 * 8 + 4 + 4 + 4 + 4  # 4 pointers, dtype, rank, scaling, padding
    assert N.Lora.scaling.offset == 4 * 8 + 8


def test_moe_lora_forward_rejects_bad_arguments():
    """e4b_moe_lora_forward validates everything before its first launch: formats, epilogues,
    ranks, shapes, dtypes and the workspace size."""
    L = N.lib()
    w1, w2 = _qw(n=128, k=64), _qw(n=64, k=64)
    lo = _lora()
    need = L.e4b_moe_lora_workspace_bytes(2, 2, 2, 128, 64, N.EPI_SWIGLU, N.BF16, 16)
    assert need >= L.e4b_moe_lora_workspace_bytes(2, 2, 2, 128, 64, N.EPI_SWIGLU, N.BF16, 1) > 0

    def call(w1=w1, w2=w2, lo=lo, epi=N.EPI_SWIGLU, ws=need, tokens=2, act=N.BF16, flags=0):
        return L.e4b_moe_lora_forward(4096, act, tokens, 4096, 4096, N.BF16, 2, ctypes.byref(w1), ctypes.byref(w2),
                                      ctypes.byref(lo) if lo is not None else None, epi, 7.0, flags, 4096, ws, 8192,
                                      N.BF16, None)

    assert call(lo=None) == -1 and "lora is NULL" in _err()
    m1, m2 = _qw(n=128, k=64, format=N.FMT_MXFP4), _qw(n=64, k=64, format=N.FMT_MXFP4)
    assert call(w1=m1, w2=m2) == -2 and "NF4" in _err()
    assert call(epi=N.EPI_GPTOSS) == -2 and "epilogue" in _err()
    assert call(epi=N.EPI_NONE) == -2 and "epilogue" in _err()
    assert call(lo=_lora(rank=0)) == -2 and "rank" in _err()
    assert call(lo=_lora(rank=65)) == -2 and "rank" in _err()
    assert call(lo=_lora(dtype=7)) == -1 and "adapter dtype" in _err()
    assert call(w2=_qw(n=64, k=128)) == -1 and "chain" in _err()
    assert call(act=N.FP32) == -1 and "act_dtype" in _err()
    assert call(flags=9) == -1 and "flags" in _err()
    assert call(ws=need - 1) == -4 and "workspace" in _err()
    assert call(tokens=0, ws=0) == 0  # no tokens: a valid no-op


def test_lora_workspace_covers_both_paths():
    L = N.lib()
    for T in (1, 8, 64, 4096):
        got = L.e4b_moe_lora_workspace_bytes(T, 8, 64, 2048, 2048, N.EPI_SWIGLU, N.BF16, 64)
        M = T * 8
        decode = M * 1024 * 2 + 2 * M * 64 * 4
        grouped = M * (2048 * 4 + 1024 * 2 + 2048 * 4 + 64 * 4)
        assert got >= max(decode, grouped), T


def test_workspace_grows_with_tokens():
    L = N.lib()
    a = L.e4b_moe_workspace_bytes(1, 8, 64, 2048, 2048, N.EPI_SWIGLU, N.BF16)
    b = L.e4b_moe_workspace_bytes(4096, 8, 64, 2048, 2048, N.EPI_SWIGLU, N.BF16)
    assert b > a and b >= 4096 * 8 * (1024 + 2048) * 2


def test_native_error_raises_with_message():
    with pytest.raises(N.NativeError, match="status -1"):
        N.lib().e4b_dequant(None, 0, 1, N.FP32, 4096, None)
        N.check("e4b_dequant", -1)


def test_descriptor_structs_follow_field_changes():
    """QW caches its C struct; assigning a field (a bias added after a first call, say) must
    rebuild the struct, never hand the library a stale pointer."""
    import torch
    from experts4bit_qlora_amd import ops

    qw = ops.QW(N.FMT_MXFP4, 2, 64, 64, torch.zeros(2 * 64 * 32, dtype=torch.uint8),
                torch.zeros(2 * 64 * 2, dtype=torch.uint8))
    s1 = qw.struct()
    assert qw.struct() is s1 and not s1.bias
    bias = torch.ones(2, 64)
    qw.bias = bias
    s2 = qw.struct()
    assert s2 is not s1 and s2.bias == bias.data_ptr()


def _header_fields(struct):
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(rf"typedef struct {struct} \{{(.*?)\}} {struct};", src, flags=re.S).group(1)
    return re.findall(r"(\w+)\s*;", body)


def _integration_binding():
    """Execute the reference-side ctypes binding documented in INTEGRATION.md (its library path
    pointed at the built library) and return its namespace."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    snippet = next(b for b in blocks if "class QWeight" in b)
    path = re.search(r'ctypes\.CDLL\("([^"]+)"\)', snippet).group(1)
    ns = {}
    exec(compile(snippet.replace(path, N.LIB_PATH), "INTEGRATION.md", "exec"), ns)
    return ns


def test_integration_binding_matches_header_and_native():
    """The binding a maintainer copies from INTEGRATION.md must lay out e4b_qweight exactly as the
    header and _native do: a short struct would make the library read past its end."""
    ns = _integration_binding()
    doc = ns["QWeight"]
    names = [f[0] for f in doc._fields_]
    assert names == [f[0] for f in N.QWeight._fields_] == _header_fields("e4b_qweight")
    assert [f[1] for f in doc._fields_] == [f[1] for f in N.QWeight._fields_]
    assert ctypes.sizeof(doc) == ctypes.sizeof(N.QWeight)
    for name, _ in doc._fields_:
        assert getattr(doc, name).offset == getattr(N.QWeight, name).offset, name

    def norm(types):  # POINTER(<doc QWeight>) and POINTER(N.QWeight) compare by their layout
        out = []
        for t in types:
            base = getattr(t, "_type_", None)
            out.append(("ptr", tuple(base._fields_)) if isinstance(base, type) and
                       issubclass(base, ctypes.Structure) else t)
        return out

    L, D = N.lib(), ns["_lib"]
    for fn in ("e4b_moe_forward", "e4b_moe_workspace_bytes"):
        assert norm(getattr(D, fn).argtypes) == norm(getattr(L, fn).argtypes), fn
        assert getattr(D, fn).restype == getattr(L, fn).restype, fn

    # the documented descriptor helper fills every field (shift left NULL: no fp16 mode)
    import torch

    class _Mod:
        num_experts = 4
        code = torch.zeros(16)

    pk, am = torch.zeros(64, dtype=torch.uint8), torch.zeros(8)
    q = ns["_qw"](_Mod(), pk, am, 32, 64)
    assert (q.format, q.num_experts, q.n, q.k) == (ns["NF4"], 4, 32, 64)
    assert q.packed == pk.data_ptr() and q.absmax == am.data_ptr() and q.code == _Mod.code.data_ptr()
    assert not q.shift and not q.bias and not q.absmax2


def test_routing_and_lora_structs_match_header():
    assert [f[0] for f in N.Routing._fields_] == _header_fields("e4b_routing")
    assert [f[0] for f in N.Lora._fields_] == _header_fields("e4b_lora")
