"""The single-token decode launch (decode_fused_kernel: e4b_moe_forward at tokens == 1 with
E4B_PATH_DECODE_FUSED).

Every block of one launch computes a slice of gate_up, hands its h to the other blocks through
an exchange buffer the library owns (zero until written; consumers read until no value is
zero), then computes a slice of down and the combine. These tests hold its layer output against
the fp64 oracle over the oracle-decoded weights (relative Frobenius <= 1e-2, max-abs <= 2e-2 of
the output RMS), and against the two-launch decode path on the same inputs; they cover ragged
chunk counts, every expert routed (several gate_up passes and down job passes per block), more
down columns than one pass of the grid, invalid and duplicated expert ids, repeated calls on
several streams (each stream's buffers alternate from call to call), graph replays, and a wait
that gives up (forced from the host with a one-tick limit) followed by correct calls.
"""
import numpy as np
import pytest
import torch

from decode_layers import Layer as _Layer, _check, _inputs
from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import ops
from oracle import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"


class Layer(_Layer):
    """A layer whose run() defaults to the single-launch path."""

    def run(self, x, idx, wts, path=N.PATH_DECODE_FUSED, out_dtype=torch.float32):
        return super().run(x, idx, wts, path=path, out_dtype=out_dtype)


def _announce(msg):
    print(f"[case] {msg}", flush=True)


_CASES = [  # fmt, E, H, I, top, dt
    ("nf4", 16, 2048, 1024, 8, torch.bfloat16),     # OLMoE rows (64 + 32 chunks)
    ("nf4", 8, 768, 320, 2, torch.bfloat16),        # ragged: 24 / 10 chunks over 8 / 32 lanes
    ("nf4", 8, 768, 320, 2, torch.float16),
    ("nf4_dq", 8, 768, 320, 2, torch.bfloat16),
    ("nf4_dq", 8, 768, 320, 2, torch.float16),
    ("mxfp4", 8, 768, 320, 2, torch.bfloat16),
    ("mxfp4", 8, 768, 320, 2, torch.float16),
    ("nf4_dq", 16, 2048, 768, 8, torch.bfloat16),   # Qwen3 rows
    ("mxfp4", 8, 2880, 2880, 4, torch.bfloat16),    # gpt-oss rows: 90 down chunks, 3 per lane
    ("nf4", 32, 2048, 512, 32, torch.bfloat16),     # every expert routed: 2 gate_up passes, 4 job passes
    ("nf4", 4, 4096, 256, 4, torch.float16),        # 4096 down columns: 2 column tiles per block
]


@pytest.mark.parametrize("fmt,E,H,I,top,dt", _CASES)
def test_single_launch_decode_matches_oracle_and_two_launch_path(fmt, E, H, I, top, dt):
    _announce(f"fused decode fmt={fmt} E={E} H={H} I={I} top={top} dt={dt}")
    L = Layer(fmt, E, H, I, dt)
    for seed in (70, 71):
        x, idx, wts = _inputs(E, H, top, seed, dt)
        fused = L.run(x, idx, wts)
        split = L.run(x, idx, wts, path=N.PATH_AUTO)
        want = L.oracle(x, idx, wts)
        _check(fused, want, "fused")
        _check(split, want, "two-launch")
        fro, maxabs, _ = moe.rel_errors(fused.cpu().numpy(), split.cpu().numpy().astype(np.float64))
        assert fro <= 5e-3 and maxabs <= 1e-2, ("fused vs two-launch", fro, maxabs)
        for od in (torch.bfloat16, torch.float16):  # output rounded once from the same fp32 sums
            o = L.run(x, idx, wts, out_dtype=od)
            assert o.dtype == od and torch.equal(o, fused.to(od))
    assert ops.decode_sync_errors() == 0


def test_invalid_duplicate_and_unrouted_ids():
    """Ids outside [0, E) drop their slot; a repeated id gives each of its slots the expert's
    output under that slot's weight; with no valid id the output is zero."""
    _announce("fused decode invalid / duplicate ids")
    E, H, I = 8, 768, 320
    L = Layer("nf4", E, H, I, torch.bfloat16)
    for ids in ([[3, -1, 8, 5]], [[2, 2, 6, 2]], [[-5, 9, 100, -1]], [[7]]):
        x, idx, wts = _inputs(E, H, len(ids[0]), 80, torch.bfloat16, ids=ids)
        fused = L.run(x, idx, wts)
        split = L.run(x, idx, wts, path=N.PATH_AUTO)
        want = L.oracle(x, idx, wts)
        if not np.any(want):
            assert not torch.any(fused) and not torch.any(split), ids
            continue
        _check(fused, want, ("fused", ids))
        _check(split, want, ("two-launch", ids))
    assert ops.decode_sync_errors() == 0


def test_repeated_calls_on_several_streams():
    """The launch counters are never reset: every call derives its buffer parity from the counts
    it finds. Calls alternate between the default stream and two side streams (each stream has
    its own counters and buffers), with a different token each time."""
    _announce("fused decode repeated calls / streams")
    E, H, I, top = 16, 2048, 1024, 8
    L = Layer("nf4", E, H, I, torch.bfloat16)
    streams = [torch.cuda.current_stream(), torch.cuda.Stream(), torch.cuda.Stream()]
    inputs = [_inputs(E, H, top, 90 + i, torch.bfloat16) for i in range(9)]
    wants = [L.run(x, idx, wts, path=N.PATH_AUTO) for x, idx, wts in inputs]
    torch.cuda.synchronize()
    outs = []
    for i, (x, idx, wts) in enumerate(inputs):
        s = streams[i % 3]
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            outs.append(L.run(x, idx, wts))
    torch.cuda.synchronize()
    for i, (o, w) in enumerate(zip(outs, wants)):
        fro, maxabs, _ = moe.rel_errors(o.cpu().numpy(), w.cpu().numpy().astype(np.float64))
        assert fro <= 5e-3 and maxabs <= 1e-2, (i, fro, maxabs)
    assert ops.decode_sync_errors() == 0


def test_graph_replays_match_eager():
    """The launch captured in a graph and replayed with new inputs copied in between: every
    replay equals the eager call on the same inputs, bit for bit."""
    _announce("fused decode graph replay")
    E, H, I, top = 16, 2048, 1024, 8
    L = Layer("nf4", E, H, I, torch.bfloat16)
    x, idx, wts = _inputs(E, H, top, 100, torch.bfloat16)
    L.run(x, idx, wts)  # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = L.run(x, idx, wts)
    for i in range(4):
        xi, ii, wi = _inputs(E, H, top, 101 + i, torch.bfloat16)
        x.copy_(xi)
        idx.copy_(ii)
        wts.copy_(wi)
        g.replay()
        torch.cuda.synchronize()
        eager = L.run(xi, ii, wi)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
    assert ops.decode_sync_errors() == 0


def test_wait_that_gives_up_raises_the_flag_and_later_calls_are_right():
    """With a one-tick wait limit (set from the host), blocks that find h unfinished stop
    waiting: the kernel still ends normally, the sticky flag records it (when it happened) and
    the call's output is undefined. Every block still announces its h exactly once, so calls
    after the limit is restored wait correctly and match the two-launch path."""
    _announce("fused decode wait limit")
    E, H, I, top = 16, 2048, 1024, 8
    L = Layer("nf4", E, H, I, torch.bfloat16)
    x, idx, wts = _inputs(E, H, top, 110, torch.bfloat16)
    want = L.run(x, idx, wts, path=N.PATH_AUTO)
    ops.decode_sync_errors(reset=True)
    try:
        ops.decode_wait_limit(1)
        for _ in range(3):
            L.run(x, idx, wts)
        torch.cuda.synchronize()
        flagged = ops.decode_sync_errors(reset=True)
        assert flagged in (0, 1)
    finally:
        ops.decode_wait_limit(0)
    for _ in range(3):
        got = L.run(x, idx, wts)
        fro, maxabs, _ = moe.rel_errors(got.cpu().numpy(), want.cpu().numpy().astype(np.float64))
        assert fro <= 5e-3 and maxabs <= 1e-2, (fro, maxabs)
    assert ops.decode_sync_errors() == 0


def test_single_launch_is_what_runs():
    """With the fused flag one token's layer is one kernel launch (decode_fused_kernel); the
    two-launch decode path (forced with E4B_PATH_GEMV) runs the up and down kernels."""
    _announce("fused decode launch count")
    E, H, I, top = 8, 768, 320, 2
    L = Layer("nf4", E, H, I, torch.bfloat16)
    x, idx, wts = _inputs(E, H, top, 120, torch.bfloat16)
    L.run(x, idx, wts)
    torch.cuda.synchronize()
    from torch.profiler import ProfilerActivity, profile

    def kernels(path):
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            L.run(x, idx, wts, path=path)
            torch.cuda.synchronize()
        return [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]

    fused, split = kernels(N.PATH_DECODE_FUSED), kernels(N.PATH_GEMV)
    if not fused and not split:
        pytest.skip("the profiler recorded no device activity on this system")
    assert sum("decode_fused_kernel" in n for n in fused) == 1, fused
    assert not any("decode_up_kernel" in n or "decode_down_kernel" in n for n in fused), fused
    assert any("decode_up_kernel" in n for n in split) and any("decode_down_kernel" in n for n in split), split
