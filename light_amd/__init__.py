"""light_amd: MI355X-native (gfx950) quantized-weight matmul path for Light.

* ``light_amd.hipq``  -- ctypes binding of libhipq's C ABI (include/hipq.h).
* ``light_amd.synth`` -- seeded synthetic inputs of the benchmark configurations.
* ``light_amd.build`` -- hipcc build of libhipq.so.
"""
__all__ = ["hipq", "synth", "build"]
