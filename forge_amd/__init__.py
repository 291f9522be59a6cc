"""forge_amd: MI355X (gfx950) quantized-matmul hot path for Forge.

The product is the shared library ``libforge_q.so`` (C ABI in
include/forge_q.h) built from ``forge_amd/csrc``.  ``forge_amd.ops`` mirrors
Forge's operator API over it; ``forge_amd.formats`` and ``forge_amd.synth``
describe the block formats and make seeded synthetic inputs.
"""
from . import formats  # noqa: F401

__all__ = ["formats"]
