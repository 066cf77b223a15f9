"""nanokv_amd -- MI355X (gfx950) implementation of NanoKV's codec-native
historical attention: INT4 chunk codec, fused decode+attention and the
NanoKV-Fast mixed-dimensional read, behind the reference's Python API.

Submodules:
  ops           torch-facing wrappers of the HIP kernels (C ABI, include/nanokv.h)
  nanokv_codec  the reference codec API (encode_tensor, decode_value, ...)
  codec_native  partition attention, LSE merge, readers and the attention hook
  synth         seeded synthetic inputs of the benchmark shapes
  build         in-tree hipcc build of libnanokv_hip.so
"""
__all__ = ["ops", "synth", "build"]
