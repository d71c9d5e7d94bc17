"""rgpu_amd: MI355X (gfx950) training backend for rtensor's MLP step.

The product is librtensor_hip.so (HIP kernels + C ABI, include/rtensor_hip.h);
``rgpu_amd.gpu`` mirrors the ``rtensor::gpu`` API over that ABI.
"""
from .gpu import Gpu, GpuMlp, GpuTensor, RtError, upload_labels  # noqa: F401
