"""Prefill-size forwards issued from several host threads at once.

A prefill-size ``e4b_moe_forward`` runs its 32-row tail tiles on a second stream, forked from and
joined back to the caller's stream with events inside the call. These tests run different inputs
through ONE module from two host threads, each on its own stream (ctypes releases the GIL inside
the library, so the enqueues interleave), and require every result to equal, bit for bit, what a
single thread computed for the same input. A fork or join event shared between threads would let
one call's tail tiles start before its routing or scaled tokens exist, or let its combine start
before its tail tiles ended. The last test also captures one thread's forward into a HIP graph
while the other thread runs eagerly.
"""
import threading

import pytest
import torch

import experts4bit_qlora_amd as e4b
from experts4bit_qlora_amd import fast as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _module(E=16, H=512, inter=256, dq=False, seed=5):
    g = torch.Generator().manual_seed(seed)
    gu = torch.randn(E, 2 * inter, H, generator=g) * 0.05
    dn = torch.randn(E, H, inter, generator=g) * 0.05
    mod = e4b.Experts4bit.from_float(gu.to(DEV), dn.to(DEV), compute_dtype=torch.bfloat16,
                                     compress_statistics=dq).eval()
    assert e4b.enable_fast(mod) == 1
    return mod


def _inputs(T, E, H, k, seed):
    """Zipf(1.1)-skewed routing, so head experts fill 256-row tiles and the tail experts end in
    32-row tiles (the side-stream launches)."""
    g = torch.Generator().manual_seed(seed)
    rank = torch.randperm(E, generator=g).float() + 1.0
    logits = torch.randn(T, E, generator=g) - 1.1 * torch.log(rank)
    val, idx = torch.topk(torch.softmax(logits, -1), k, dim=-1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    return x.to(DEV), idx.to(DEV), val.to(torch.bfloat16).to(DEV)


def _run_threads(jobs):
    """Run each job(barrier, errors) in its own thread; return the error list."""
    errors = []
    barrier = threading.Barrier(len(jobs))
    threads = [threading.Thread(target=j, args=(barrier, errors)) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
        assert not t.is_alive(), "a thread did not finish"
    return errors


def _eager_job(mod, inp, ref, reps, label):
    def job(barrier, errors):
        try:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(stream), torch.no_grad():
                barrier.wait()
                outs = [mod(*inp) for _ in range(reps)]
            stream.synchronize()
            for i, o in enumerate(outs):
                if not torch.equal(o, ref):
                    errors.append(f"{label}: call {i} differs from the single-thread result "
                                  f"(max |diff| {(o.float() - ref.float()).abs().max().item():.3e})")
                    return  # the first mismatch is enough
        except Exception as exc:  # reported by the main thread
            errors.append(f"{label}: {exc!r}")
    return job


@pytest.mark.parametrize("dq", [False, True])
def test_two_threads_prefill_match_single_thread(dq):
    E, H, inter, k = 16, 512, 256, 4
    _announce(f"two host threads, prefill-size forwards, dq={dq}")
    mod = _module(E, H, inter, dq=dq, seed=5 + dq)
    a = _inputs(512, E, H, k, seed=11)
    b = _inputs(384, E, H, k, seed=12)
    with torch.no_grad():
        ref_a, ref_b = mod(*a), mod(*b)
    torch.cuda.synchronize()
    assert F._qweights(mod)[0].shift is not None  # the fp16 mode: 256-row + 32-row tiles
    errors = _run_threads([_eager_job(mod, a, ref_a, 12, "thread A"), _eager_job(mod, b, ref_b, 12, "thread B")])
    assert not errors, errors


def test_capture_in_one_thread_eager_in_another():
    """One thread captures a prefill-size forward into a HIP graph while another thread issues
    eager forwards on its own stream: the eager calls must not use a second stream that the
    capture holds, and the graph's replays must equal the eager result."""
    E, H, inter, k = 16, 512, 256, 4
    _announce("capture in one thread, eager forwards in another")
    mod = _module(E, H, inter, seed=9)
    a = _inputs(512, E, H, k, seed=21)
    b = _inputs(448, E, H, k, seed=22)
    with torch.no_grad():
        ref_a, ref_b = mod(*a), mod(*b)
    torch.cuda.synchronize()
    graphs = {}

    def capture_job(barrier, errors):
        try:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.default_stream())
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(stream), torch.no_grad():
                barrier.wait()
                with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
                    out = mod(*a)
            graphs["a"] = (g, out)
        except Exception as exc:
            errors.append(f"capture thread: {exc!r}")

    errors = _run_threads([capture_job, _eager_job(mod, b, ref_b, 12, "eager thread")])
    assert not errors, errors
    g, out = graphs["a"]
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_a), f"replay {rep} differs from the eager result"
        # eager work between replays
        with torch.no_grad():
            again = mod(*b)
        torch.cuda.synchronize()
        assert torch.equal(again, ref_b)


def test_probe_events_time_each_prefill_launch_without_changing_results():
    """e4b_set_probe: while a site is set the forward runs both tile heights on the caller's
    stream and records the caller's event pair around the watched launch. Each site yields a
    positive duration shorter than the whole forward, the probed forward's output equals the
    unprobed (two-stream) one bit for bit, and clearing the probe leaves later forwards
    unrecorded (the pair keeps its last timestamps)."""
    from experts4bit_qlora_amd import _native as N

    L = N.lib()
    mod = _module()
    x, idx, w = _inputs(2048, 16, 512, 4, seed=31)
    with torch.no_grad():
        ref = mod(x, idx, w)
    before, after = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    before.record()
    after.record()
    torch.cuda.synchronize()
    for site in (N.PROBE_GATE_UP_BIG, N.PROBE_GATE_UP_TAIL, N.PROBE_DOWN_BIG, N.PROBE_DOWN_TAIL):
        _announce(f"probe site {site}")
        torch.cuda._sleep(100_000)
        N.check("e4b_set_probe", L.e4b_set_probe(site, before.cuda_event, after.cuda_event))
        try:
            start.record()
            with torch.no_grad():
                out = mod(x, idx, w)
            end.record()
        finally:
            N.check("e4b_set_probe", L.e4b_set_probe(N.PROBE_OFF, None, None))
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"site {site}: the probed forward differs"
        t_launch, t_all = before.elapsed_time(after), start.elapsed_time(end)
        assert 0.0 < t_launch < t_all, (site, t_launch, t_all)
    # cleared: a forward records nothing, so the pair still spans the last probed launch
    last = before.elapsed_time(after)
    with torch.no_grad():
        mod(x, idx, w)
    torch.cuda.synchronize()
    assert before.elapsed_time(after) == last
    with pytest.raises(N.NativeError):
        N.check("e4b_set_probe", L.e4b_set_probe(7, None, None))
