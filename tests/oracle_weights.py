"""Oracle-side weights for the GPU parity tests: a module's stored bytes decoded on the CPU by
the oracle's C restatement (``oracle/c/oracle.c``, pinned against the numpy restatement in
``tests/test_oracle.py``), never by the HIP dequant kernel under test."""
from oracle import c_oracle


class OracleExperts:
    """``[E, n, k]`` fp32 weights of one projection, decoded per expert on first use.

    ``fmt``: ``"nf4"`` (fp32 absmax), ``"nf4_dq"`` (u8 codes + absmax2 + offset + code2) or
    ``"mxfp4"`` (e8m0 scales). Indexing returns the ``[n, k]`` fp32 array of one expert."""

    def __init__(self, mod, which: str, fmt: str):
        self.n, self.k = mod._gate_up_shape if which == "gate_up" else mod._down_shape
        E = mod.num_experts
        self.shape = (E, self.n, self.k)
        self.fmt = fmt
        self.packed = getattr(mod, f"{which}_proj").detach().cpu().numpy().reshape(E, -1)
        self.absmax = getattr(mod, f"{which}_absmax").detach().cpu().numpy().reshape(E, -1)
        if fmt == "nf4_dq":
            self.absmax2 = getattr(mod, f"{which}_absmax2").detach().cpu().numpy().reshape(E, -1)
            self.offset = getattr(mod, f"{which}_absmax_offset").detach().cpu().numpy().reshape(E)
            self.code2 = mod.code2.detach().cpu().numpy()
        if fmt != "mxfp4":
            self.code = mod.code.detach().cpu().numpy()
        self._cache = {}

    def __getitem__(self, e):
        e = int(e)
        if e not in self._cache:
            if self.fmt == "mxfp4":
                v = c_oracle.dequant_mxfp4(self.packed[e], self.absmax[e], self.n, self.k)
            else:
                am = self.absmax[e]
                if self.fmt == "nf4_dq":
                    am = c_oracle.dequant_absmax_dq(am, self.absmax2[e], self.offset[e], self.code2)
                v = c_oracle.dequant_4bit(self.packed[e], am, self.code)
            self._cache[e] = v.reshape(self.n, self.k)
        return self._cache[e]


def module_format(mod) -> str:
    from experts4bit_qlora_amd.arch.gptoss import GptOssExpertsMxfp4

    if isinstance(mod, GptOssExpertsMxfp4):
        return "mxfp4"
    return "nf4_dq" if getattr(mod, "compress_statistics", False) else "nf4"


def oracle_weights(mod):
    fmt = module_format(mod)
    return OracleExperts(mod, "gate_up", fmt), OracleExperts(mod, "down", fmt)
