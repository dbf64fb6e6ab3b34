"""FP32 nonlinearities at the MoE rounding boundaries (test oracle only).

Follows ``kaggle/qwen38_tpu/numerics.py:13-51`` (accurate exp, corrected
divide, sigmoid, softmax) and ``kaggle/qwen38_tpu/math.py:19-24`` (silu with
an explicit BF16 boundary). exp is evaluated in FP64 and rounded once to FP32;
each division is one correctly rounded FP32 division, which is what the
reference's residual-corrected quotient approximates.
"""

import numpy as np

from .packed_q6 import bf16_round


def exp_f32(x):
    return np.exp(np.asarray(x, np.float64)).astype(np.float32)


def sigmoid(x):
    """numerics.py:42-45: e = exp(-|x|); where(x >= 0, 1, e) / (1 + e), in FP32."""
    x = np.asarray(x, np.float32)
    e = exp_f32(-np.abs(x))
    num = np.where(x >= 0, np.float32(1), e).astype(np.float32)
    return (num / (np.float32(1) + e)).astype(np.float32)


def silu_bf16(x):
    """math.py:19-20: RNE_bf16(f32(x) * sigmoid(x)) for BF16-valued x."""
    x = np.asarray(x, np.float32)
    return bf16_round(x * sigmoid(x))


def softmax(x, axis=-1):
    """numerics.py:48-51: exp(x - max) / sum, in FP32."""
    x = np.asarray(x, np.float32)
    e = exp_f32(x - np.max(x, axis=axis, keepdims=True))
    return (e / np.sum(e, axis=axis, keepdims=True, dtype=np.float32)).astype(np.float32)
