"""qwenasr_amd — MI355X (gfx950) HIP backend for QwenASR's int8 inference hot path.

The product is libqasr_hip.so (C ABI in include/qasr_hip.h).  This package is
the host-side mirror of the reference's operator API over that ABI:

    qwenasr_amd.kernels  kernels:: int8 ops (quantizers, matvecs, argmax, norms,
                         RoPE, attention) on device arrays
    qwenasr_amd.model    Decoder (Decoder::load + KvCache + prefill/forward)
    qwenasr_amd.synth    seeded synthetic weights / audio for benches and tests
"""
from ._lib import QASR_ROUND_HALF_AWAY, QASR_TRUNC, QasrError, lib  # noqa: F401
from .device import Device, DeviceArray, device_count  # noqa: F401
