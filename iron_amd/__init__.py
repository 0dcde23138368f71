"""iron_amd: MI355X-native (gfx950) Qwen3 int8 decode hot path with IRON's operator API.

Compute runs only in ``libiron_hip.so`` (hand-written HIP kernels behind the C ABI in
``include/iron_hip.h``); Python mirrors the reference's operator, sequence and application
interfaces on top of it.
"""

__version__ = "0.1.0"
