"""kansaiml_amd -- an MI355X (gfx950) HIP backend for Kansai's int8
quantize -> int8 matmul -> dequantize path and its fp32 matmul.

Modules:
  _native   ctypes binding of the C ABI (include/kansai_hip.h)
  device    DeviceTensor: pooled device buffers
  hip       tensor-level ops (shape checks + kernel calls)
  quantize  the reference's quantize.py API on the GPU
  kir       the KIR graph schema, tracer, memory planner and run_hip
  serialize KAN1 parameter checkpoints, with int8 weights that load
            straight to the device
  charlm    the int8 char-LM forward (config C4)
  build     compiles kansaiml_amd/csrc/*.hip for gfx950

Importing the package does not touch the GPU.
"""

__all__ = ["available"]


def available() -> bool:
    from . import _native
    return _native.available()
