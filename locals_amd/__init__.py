"""locals_amd: MI355X (gfx950) drop-in for Locals' batched attention hot path.

Modules mirror the reference's call surface (Generated-Computers/Locals):

* ``locals_amd.qkv``        <- locals/qkv.py        (8-bit KV split-K decode, caches, quantize)
* ``locals_amd.attention``  <- locals/attention.py  (ragged fp16/bf16 decode)

Every function runs hand-written HIP kernels from ``liblocals_amd.so`` (C ABI: include/locals_amd.h) on torch's
current stream; there is no CPU fallback.
"""

from . import _lib  # noqa: F401

__all__ = ["qkv", "attention"]
