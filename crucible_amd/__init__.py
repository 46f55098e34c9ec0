"""crucible_amd: MI355X (gfx950) attention hot path of the crucible inference engine.

The product is ``libcrucible_attn.so`` (C ABI: include/crucible_attn.h), hand-written
HIP for paged decode, causal and packed prefill, and the fp16 KV append. This package
holds its sources (``csrc/``), the build (``_build``), the ctypes binding (``_lib``), the
host mirror of the reference's launch API (``gpu.Gpu``), paging bookkeeping (``paged``)
and the synthetic workloads of the benchmark configs (``workloads``).
"""
from ._lib import CrucibleError, load  # noqa: F401

__all__ = ["CrucibleError", "load"]
