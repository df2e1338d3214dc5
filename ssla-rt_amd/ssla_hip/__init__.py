"""ssla_hip: host side of the MI355X drain of SSLA-S s2 + s3 + YOLOX head.

  abi     numpy / ctypes mirrors of include/ssla_abi.h
  lib     ctypes binding of libssla_hip.so (include/ssla_hip.h)
  hybrid  device buffers, weight packing, HybridS2S3Config, drain calls
  stub    weight-directory generator (tools/make_ssla_stub.py schema)
  events  seeded synthetic event / ring-record streams
"""
from . import abi, events, stub  # noqa: F401  (no GPU needed)

__all__ = ["abi", "events", "stub", "lib", "hybrid"]
