"""The sync-free decode engine pieces: the device-id grouped call, the address-table row gather,
and a captured 16-layer decode step replayed under torch's sync-debug "error" mode.

Contracts (reference): the device-id grouped call of engines/pipelined.py:502-508 (fixed host
sizes, ids as a device tensor, no read-back); the gather of pipelined.py:117-151 (per-slot
absolute source address, identity-based skip) with its traffic accounting (:471-487); the
zero-sync token loop of tests/test_pipelined.py:113-133.
"""
import numpy as np
import pytest
import torch

import experts4bit_qlora_amd as e4b
from experts4bit_qlora_amd import _native as N
from experts4bit_qlora_amd import ops, quant as Q
from oracle import c_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _nf4(E, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    packed, absmax = Q.quantize_4bit(torch.randn(E, n * k, generator=g) * 0.05)
    return packed.view(E, n, k // 2).to(DEV), absmax.view(E, n, k // 64).to(DEV)


def _dense(packed, absmax):
    code = Q.code_4bit("nf4").numpy()
    E, n, kh = packed.shape
    return np.stack([c_oracle.dequant_4bit(packed[e].reshape(-1).cpu().numpy(), absmax[e].reshape(-1).cpu().numpy(),
                                           code).reshape(n, 2 * kh) for e in range(E)])


@pytest.mark.parametrize("sizes", [[3, 0, 5, 1], [1] * 8, [40, 70, 9], [130, 0, 300]])
def test_device_id_grouped_call_equals_the_host_list_call(sizes):
    """Ascending distinct ids (the host-list call's domain): both calls give the same rows, bit
    for bit, and the device one never reads the ids back."""
    _announce(f"device-id grouped call sizes={sizes}")
    E, n, k = 8, 192, 256
    w, am = _nf4(E, n, k, 1)
    ids = sorted(np.random.default_rng(len(sizes)).permutation(E)[:len(sizes)].tolist())
    a = torch.randn(sum(sizes), k, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    host = ops.gemm_4bit_grouped(a, w, am, sizes, ids)
    dev_ids = torch.tensor(ids, device=DEV)
    ops.gemm_4bit_grouped(a, w, am, sizes, dev_ids)  # warm the allocator
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        dev = ops.gemm_4bit_grouped(a, w, am, sizes, dev_ids)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    assert torch.equal(host, dev)


def test_device_ids_in_any_order_repeated_and_out_of_range():
    """Unsorted, repeated and out-of-range ids (the slot rows of a residency engine need not be
    ordered): each group's rows are its expert's projection against the oracle-decoded weights
    (fp32 output rows, within GEMM rounding), rows of an out-of-range id are zero, and the result
    equals the same groups run one at a time bit for bit."""
    _announce("device ids unordered / repeated / out of range")
    E, n, k = 8, 192, 256
    w, am = _nf4(E, n, k, 3)
    W = _dense(w, am).astype(np.float64)
    sizes, ids = [6, 5, 0, 7, 5, 9], [6, 1, 6, 9, -2, 0]  # >= 5 rows: every call takes the MFMA path
    a = torch.randn(sum(sizes), k, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    got = ops.gemm_4bit_grouped(a, w, am, sizes, torch.tensor(ids, device=DEV)).float().cpu().numpy()
    r = 0
    for s, e in zip(sizes, ids):
        rows = got[r:r + s]
        if s == 0:
            continue
        if 0 <= e < E:
            want = a[r:r + s].float().cpu().numpy().astype(np.float64) @ W[e].T
            assert np.abs(rows - want).max() <= 1e-2 * max(np.abs(want).max(), 1e-6) + 1e-3, (e, s)
            one = ops.gemm_4bit_grouped(a[r:r + s], w, am, [s], torch.tensor([e], device=DEV))
            assert np.array_equal(rows, one.float().cpu().numpy()), (e, s)
        else:
            assert not np.any(rows), (e, s)
        r += s


def test_route_groups_tables():
    """offsets / active / tiles / meta / sorted_flat / inv of the device group routing against a
    host restatement of the same rule."""
    _announce("route_groups tables")
    E, tm = 6, 4
    sizes, ids = [5, 3, 0, 2, 7, 1], [4, 1, 4, 7, 0, 1]
    rb = ops.route_groups(sizes, torch.tensor(ids, device=DEV), E, tile_m=tm)
    torch.cuda.synchronize()
    off = np.concatenate([[0], np.cumsum(sizes)])
    cnt = np.zeros(E, int)
    for s, e in zip(sizes, ids):
        if 0 <= e < E:
            cnt[e] += s
    starts = np.concatenate([[0], np.cumsum(cnt)])
    inv = np.full(off[-1], -1)
    pos = starts[:-1].copy()
    for g, (s, e) in enumerate(zip(sizes, ids)):
        if 0 <= e < E:
            inv[off[g]:off[g + 1]] = np.arange(pos[e], pos[e] + s)
            pos[e] += s
    meta = rb.meta.cpu().numpy()
    assert rb.offsets.cpu().numpy().tolist() == starts.tolist()
    active = [e for e in range(E) if cnt[e] > 0]
    assert meta[1] == len(active) and rb.active.cpu().numpy()[:len(active)].tolist() == active
    assert meta[2] == sum(s for s, e in zip(sizes, ids) if not 0 <= e < E) and meta[3] == tm
    tiles = [(e, starts[e] + t * tm) for e in active for t in range(-(-cnt[e] // tm))]
    assert meta[0] == len(tiles) and rb.tiles.cpu().numpy()[:2 * len(tiles)].reshape(-1, 2).tolist() == \
        [list(t) for t in tiles]
    got_inv = rb.inv.cpu().numpy()[:off[-1]]
    assert got_inv.tolist() == inv.tolist()
    sf = rb.sorted_flat.cpu().numpy()
    for row, p in enumerate(inv):
        if p >= 0:
            assert sf[p] == row


@pytest.mark.parametrize("n_bytes,dst_off", [(4096, 0), (1000, 24), (777, 5), (3 * 65536 + 48, 16)])
def test_gather_rows_copies_and_skips(n_bytes, dst_off):
    """Slots whose wanted row differs from the one they hold receive n_bytes from the row's
    absolute address (16-byte, 8-byte and byte-granular paths; several 64 KB chunks); slots that
    already hold it are left untouched; the byte counter adds exactly the bytes moved."""
    _announce(f"gather_rows n_bytes={n_bytes} dst_off={dst_off}")
    R, k = 12, 5
    row = ((dst_off + n_bytes + 15) // 16) * 16 + 32
    arena = torch.randint(0, 256, (R, row), dtype=torch.uint8, generator=torch.Generator().manual_seed(5)).to(DEV)
    slots = torch.full((k, row), 7, dtype=torch.uint8, device=DEV)
    want = torch.tensor([3, 0, 11, 3, 6], device=DEV)
    have = torch.tensor([-1, 0, -1, -1, 6], device=DEV)  # slots 1 and 4 already hold their rows
    src = arena.data_ptr() + want * row
    copied = torch.zeros(1, dtype=torch.int64, device=DEV)
    ops.gather_rows(slots, src, want, have, n_bytes, dst_off, bytes_copied=copied)
    torch.cuda.synchronize()
    s, a = slots.cpu(), arena.cpu()
    for j, w_ in enumerate(want.tolist()):
        if j in (1, 4):
            assert torch.all(s[j] == 7), j
            continue
        assert torch.equal(s[j, dst_off:dst_off + n_bytes], a[w_, :n_bytes]), j
        assert torch.all(s[j, :dst_off] == 7) and torch.all(s[j, dst_off + n_bytes:] == 7), j
    assert int(copied.item()) == 3 * n_bytes


def test_gather_rows_rejects_a_segment_past_the_row():
    slots = torch.zeros(2, 64, dtype=torch.uint8, device=DEV)
    src = torch.full((2,), slots.data_ptr(), dtype=torch.int64, device=DEV)  # valid addresses regardless
    z = torch.zeros(2, dtype=torch.int64, device=DEV)
    with pytest.raises(N.NativeError, match="runs past"):
        ops.gather_rows(slots, src, z, z - 1, 60, dst_off=8)


def test_captured_decode_step_replays_bit_identically_without_syncs():
    """A 16-layer decode step (batch 1, independent layers) captured in a HIP graph: replays with
    new tokens copied in equal the eager step bit for bit, and neither the replays nor the eager
    forwards synchronise (torch's sync-debug mode raises on any synchronising call)."""
    _announce("captured 16-layer decode step")
    E, H, I, k, L = 16, 512, 256, 4, 16
    g = torch.Generator(device=DEV).manual_seed(9)
    mods = []
    for _ in range(L):
        m = e4b.Experts4bit.from_float(torch.randn(E, 2 * I, H, generator=g, device=DEV) * 0.02,
                                       torch.randn(E, H, I, generator=g, device=DEV) * 0.02,
                                       compute_dtype=torch.bfloat16).eval()
        assert e4b.enable_fast(m) == 1
        mods.append(m)

    def make(seed):
        gi = torch.Generator(device=DEV).manual_seed(seed)
        out = []
        for _ in range(L):
            x = torch.randn(1, H, generator=gi, device=DEV).to(torch.bfloat16)
            w, idx = torch.topk(torch.softmax(torch.randn(1, E, generator=gi, device=DEV), -1), k, dim=-1)
            out.append((x, idx, w.to(torch.bfloat16)))
        return out

    static = make(100)

    def step(inputs):
        with torch.no_grad():
            return [m(x, idx, w) for m, (x, idx, w) in zip(mods, inputs)]

    step(static)  # descriptors cached, allocator warm
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(static)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step(static)
    for rep in range(3):
        fresh = make(200 + rep)
        for (x, idx, w), (x2, idx2, w2) in zip(static, fresh):
            x.copy_(x2)
            idx.copy_(idx2)
            w.copy_(w2)
        torch.cuda.set_sync_debug_mode("error")
        try:
            graph.replay()
            eager = step(fresh)
        finally:
            torch.cuda.set_sync_debug_mode("default")
        torch.cuda.synchronize()
        for l, (o, e_) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e_), (rep, l)
