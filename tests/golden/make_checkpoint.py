"""Writes ``expertsnbit_nf4_checkpoint.pt``: an ExpertsNbit state_dict in the reference's on-disk
format, built from the format definition alone (no quantizer, no code of this package), with
inputs and the expected layer output. Run once; the output is data.

Format (reference ``_vendor/experts.py:236-327``): for ``Experts4bit(E, H, I)`` with
``quant_type="nf4"``, ``blocksize=64``, ``has_gate=True``:

* ``gate_up_proj`` u8 ``[E, 2I*H/2]``, ``down_proj`` u8 ``[E, H*I/2]``: per expert the ``[out, in]``
  matrix row-major, two values per byte, the FIRST value in the HIGH nibble;
* ``gate_up_absmax`` f32 ``[E, 2I*H/64]``, ``down_absmax`` f32 ``[E, H*I/64]``: one scale per 64
  consecutive values;
* ``_extra_state``: ``{"schema": 1, "quant_type", "blocksize", "has_gate", "num_experts",
  "hidden_dim", "intermediate_dim"}`` (``get_extra_state``, ``:279-289``);
* the ``code`` buffer is non-persistent (``:276``) and not in the file.

The expected output is the module forward in fp64 over the decoded weights: ``W[r, c] =
fp32(code[nib] * absmax[(r*in + c) // 64])``, ``h = silu(x W1g^T) * (x W1u^T)`` (gate rows first),
``y = h W2^T``, ``out[t] = sum_s w[t, s] * y_(t, s)``. Bytes and scales are seeded random.
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
NF4 = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)
E, H, I, T, K = 4, 128, 64, 6, 2


def decode(packed, absmax, rows, cols):
    """[rows, cols] fp32 from one expert's bytes, high nibble first."""
    hi, lo = packed >> 4, packed & 15
    nib = np.stack([hi, lo], axis=1).reshape(-1)
    scale = np.repeat(absmax, 64)
    return (NF4[nib].astype(np.float32) * scale.astype(np.float32)).reshape(rows, cols)


def main():
    rng = np.random.default_rng(20260)
    n1 = 2 * I
    gu = rng.integers(0, 256, (E, n1 * H // 2), dtype=np.uint8)
    dn = rng.integers(0, 256, (E, H * I // 2), dtype=np.uint8)
    gu_am = rng.uniform(0.02, 0.12, (E, n1 * H // 64)).astype(np.float32)
    dn_am = rng.uniform(0.02, 0.12, (E, H * I // 64)).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    x_bf16 = torch.from_numpy(x).to(torch.bfloat16)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 0.9, (T, K)).astype(np.float32)
    w_bf16 = torch.from_numpy(w).to(torch.bfloat16)

    xd = x_bf16.double().numpy()
    wd = w_bf16.double().numpy()
    out = np.zeros((T, H))
    for t in range(T):
        for s in range(K):
            e = idx[t, s]
            W1 = decode(gu[e], gu_am[e], n1, H).astype(np.float64)
            W2 = decode(dn[e], dn_am[e], H, I).astype(np.float64)
            p = W1 @ xd[t]
            g, u = p[:I], p[I:]
            h = g / (1.0 + np.exp(-g)) * u
            out[t] += wd[t, s] * (W2 @ h)

    state = {
        "gate_up_proj": torch.from_numpy(gu),
        "gate_up_absmax": torch.from_numpy(gu_am),
        "down_proj": torch.from_numpy(dn),
        "down_absmax": torch.from_numpy(dn_am),
        "_extra_state": {"schema": 1, "quant_type": "nf4", "blocksize": 64, "has_gate": True,
                         "num_experts": E, "hidden_dim": H, "intermediate_dim": I},
    }
    torch.save({"state_dict": state, "x": x_bf16, "top_k_index": torch.from_numpy(idx), "top_k_weights": w_bf16,
                "expected": torch.from_numpy(out)}, os.path.join(HERE, "expertsnbit_nf4_checkpoint.pt"))
    print("wrote", os.path.join(HERE, "expertsnbit_nf4_checkpoint.pt"))


if __name__ == "__main__":
    main()
