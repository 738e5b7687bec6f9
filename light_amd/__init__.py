"""light_amd: MI355X-native (gfx950) quantized-weight matmul path for Light.

* ``light_amd.hipq``  -- ctypes binding of libhipq's C ABI (include/hipq.h).
* ``light_amd.synth`` -- seeded synthetic inputs of the benchmark configurations.
* ``light_amd._light`` -- C++ host layer mirroring Light's ops / registry API
  (ops.MatMulQ, ops.MatMulInt4, ops.MoEGemmQ ... with ROCm kernels registered).
* ``light_amd.build`` -- in-tree build of libhipq.so and _light.
"""
__all__ = ["hipq", "synth", "build"]

# One HIP runtime per process: PyTorch-ROCm ships its own libamdhip64, and libhipq binds
# to whichever copy is loaded first.  Loading torch's first (when torch is installed)
# keeps torch tensors and libhipq/_light calls on the same runtime in mixed processes.
try:
    import torch as _torch  # noqa: F401
except ImportError:
    pass
