"""CPU oracle for the speculative-decoding verify step.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (``nanosglang_amd``)
imports this package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only to check results or as the
timed CPU baseline -- never as a fallback for the HIP kernels.

Modules (each function cites the reference file:line it restates):

* ``philox``           -- Philox4x32-10 counter-based uniforms (Salmon et al.,
                          SC'11), pinned by the Random123 known-answer vectors.
* ``page_table``       -- CSR page-table / slot arithmetic
                          (nano_sglang/engine/engine.py:419-448).
* ``verify_attention`` -- ragged multi-query paged attention with the
                          bottom-right causal rule
                          (nano_sglang/model/causal_lm.py:359-471).
* ``acceptance``       -- greedy and stochastic acceptance, textbook residual
                          resample, bonus token, KV-slot rollback
                          (nano_sglang/decode/speculative.py:130-196).
* ``sampling``         -- temperature / top-k / top-p sampling in exact
                          fixed-point arithmetic
                          (nano_sglang/engine/sampling.py:25-50, 71-88).
* ``quantization``     -- FP8 (OCP E4M3FN) per-tensor weight quantisation and
                          the dequantisation FP8Linear applies
                          (nano_sglang/decode/quantization.py:24-75), pinned
                          against torch's own float8_e4m3fn casts.
* ``model``            -- fp32 PyTorch-CPU restatement of the Qwen2/Llama
                          decoder and the speculative loop
                          (nano_sglang/model/causal_lm.py, decode/speculative.py).

Pinning status of every function is recorded in each module's docstring.
"""
