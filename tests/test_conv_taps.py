"""The implicit-im2col GEMM of the encoder's channels-last conv stem finds the
kernel tap of each 32-wide K-step by reciprocal products in float32
(csrc/k_gemm.hip, A_CONV): t = int((k0 + 16) * (1 / C)), then
ky = int((t + 0.5) * (1 / kw)).  They must equal the integer quotients for
every K-step the kernel runs; this checks them, with the kernel's float32
rounding (no fused multiply-add), for every width C = 32 ... 4096 that is a
multiple of 32 and the kernel shapes the stem and similar convolutions use.
"""
import numpy as np


def test_reciprocal_tap_quotients_are_exact():
    shapes = ((3, 3), (16, 1), (8, 1), (1, 1), (5, 5), (7, 7), (64, 1))
    for C in range(32, 4097, 32):
        rc = np.float32(1.0) / np.float32(C)
        for kh, kw in shapes:
            rkw = np.float32(1.0) / np.float32(kw)
            k0 = np.arange(0, C * kh * kw, 32, dtype=np.int64)
            t = ((k0.astype(np.float32) + np.float32(16.0)) * rc).astype(np.int64)
            assert (t == k0 // C).all(), (C, kh, kw)
            ky = ((t.astype(np.float32) + np.float32(0.5)) * rkw).astype(np.int64)
            assert (ky == t // kw).all(), (C, kh, kw)


def test_reciprocal_check_catches_a_bad_offset():
    """Without the half-step offsets the quotient drops below the integer at
    some K-steps (the check above would catch such a kernel)."""
    bad = 0
    for C in range(32, 4097, 32):
        rc = np.float32(1.0) / np.float32(C)
        k0 = np.arange(0, C * 9, 32, dtype=np.int64)
        t = (k0.astype(np.float32) * rc).astype(np.int64)
        bad += int((t != k0 // C).sum())
    assert bad > 0
