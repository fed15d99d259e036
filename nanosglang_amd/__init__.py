"""nanosglang_amd -- MI355X (gfx950) speculative-decoding verify step.

Host-side mirror of the reference's interface for the verify path
(xiehuanyi/nanoSGLang: nano_sglang/decode/speculative.py,
nano_sglang/engine/paged_kv_cache.py) over hand-written HIP kernels exposed
through the C ABI in include/nsg_spec.h (libnsg_spec.so, built in-tree by
``python -m nanosglang_amd.build``).
"""

__version__ = "0.1.0"
