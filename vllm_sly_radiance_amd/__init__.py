"""MI355X-native MXFP4 W4A8 linear-layer path (gfx950), a drop-in for the MXFP4 W4A8 path of
vllm-sly-radiance (sly/mxfp4/radiance_mxfp4.py + radiance_mxfp4_fp8.hip).

  radiance_mxfp4   custom ops radiance::mxfp4_linear[_pq] and the vLLM kernel plugin
  _native          ctypes binding of libw4a8_mxfp4.so (C ABI in include/w4a8_mxfp4.h)
  synthetic        seeded operands with the benchmark distributions
  build            hipcc recipe for the library
"""
