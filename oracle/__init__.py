"""CPU oracle for the frozen-expert MoE forward -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of every function on the
hot path that ``enable_fast`` routes ``ExpertsNbit`` / ``Experts4bit`` modules through
(pjordanandrsn/experts4bit-qlora v0.19.1). Each function cites the reference file:line it
follows. It exists to CHECK the HIP path, never to BE it:

* only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
  import, call or link anything here;
* the product package (``experts4bit_qlora_amd``) never imports it, and its fast path
  raises when the HIP library is missing instead of falling back to anything here.

Modules:

``numerics``  bf16/fp16 round-to-nearest-even helpers (numpy, bit level).
``codes``     the NF4 / FP4 4-bit code tables and the signed dynamic 8-bit map.
``quant``     NF4 blockwise quantize/dequantize, double-quant absmax, MXFP4 quantize/dequantize.
``routing``   the token->expert stable permutation (argsort / bincount / nonzero).
``moe``       the fp32 oracle forward, the fused-path restatement, and the reference
              per-expert loop (the timed CPU baseline).
``c_oracle``  ctypes loader for ``liboracle_c.so``, a C restatement of the integer and
              dequant pieces (built by ``oracle/Makefile``), used to cross-check the numpy
              restatement and to run the byte-exact checks at full configuration sizes.

Pinning status (what checks each function, so a plausible mistake fails one of them):

* NF4 code table      -- pinned: rebuilt bit-for-bit from the published normal-quantile
                         construction, plus structural invariants.
* NF4 dequant         -- pinned: hand-computed golden vectors, brute-force loop on tiny
                         inputs, whole-stack == per-expert invariant.
* double-quant absmax -- dequant given (codes, absmax2, offset, code2) pinned by closed
                         form on hand vectors; the 256-entry ``code2`` table pinned against
                         its exact rational construction (every entry within 2 fp32 ulp)
                         and hand-derived fp32 bits of every decade's first and last cell,
                         with negative controls (a grid one point short, a decade off).
                         The quantizer's byte choices only generate inputs: parity is per
                         given bytes.
* FP4 (bnb) table     -- pinned bit for bit against bitsandbytes' published CUDA decode tree.
* LoRA forward        -- ``moe.forward_lora_fp32`` (exact) and ``moe.reference_lora_loop``
                         (the reference's rounding points): pinned by closed forms on small
                         inputs (zero adapter == base oracle; rank-1 adapter == hand sum) and
                         a negative control (delta added after the activation fails).
* routers             -- ``routing.router_topk``: pinned by brute force on small inputs
                         (sorted logits, ties to the lower expert index).
* MXFP4 dequant       -- pinned: the reference's hand-checkable golden vector and golden
                         fixtures written by transformers' ``convert_moe_packed_tensors``.
* routing             -- pinned: brute force on tiny inputs and the reference's special
                         cases (empty experts, all-to-two experts, sparse hits at E=64).
* combine / epilogues -- pinned: closed forms on hand vectors and negative controls.
"""
