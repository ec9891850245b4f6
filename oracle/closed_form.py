"""TEST INFRASTRUCTURE: float64 closed forms that pin the oracle.

Each function is the textbook definition of what an xt program computes over
a whole array, written with numpy and no reference to the oracle's loops:
  softmax_rows   e^(x - max) / sum, per row          (kernels/softmax.py:13-18)
  matmul         sum_k A[m,k] B[k,n]                 (kernels/matmul.py:16)
  conv2d_nhwc    cross-correlation with zero padding (lib/xt/XTToNova.cpp:110-142)
  conv_slice     the reference's halo-slice arithmetic (lib/xt/XTToNova.cpp:110-142)
  conv_out_dim   (in + pb + pa - (d(k-1)+1)) / s + 1  (lib/nova/NovaOps.cpp:46-59)
"""

from __future__ import annotations

import numpy as np


def softmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float64) @ np.asarray(b, dtype=np.float64)


def conv2d_nhwc(x, f, pad_top, pad_left, stride=(1, 1), dilation=(1, 1), out_hw=None):
    """out[n, oh, ow, o] = sum_{kh,kw,c} x[n, oh*sh - pt + kh*dh, ow*sw - pl + kw*dw, c] * f[kh,kw,c,o]."""
    x = np.asarray(x, dtype=np.float64)
    f = np.asarray(f, dtype=np.float64)
    n, h, w, c = x.shape
    kh_n, kw_n, _, co = f.shape
    sh, sw = stride
    dh, dw = dilation
    if out_hw is None:
        out_hw = (
            (h + 2 * pad_top - (dh * (kh_n - 1) + 1)) // sh + 1,
            (w + 2 * pad_left - (dw * (kw_n - 1) + 1)) // sw + 1,
        )
    oh_n, ow_n = out_hw
    # pad generously, then gather each tap as a strided view
    big = max(kh_n * dh, kw_n * dw) + max(sh, sw) * max(oh_n, ow_n)
    xp = np.zeros((n, h + pad_top + big, w + pad_left + big, c))
    xp[:, pad_top : pad_top + h, pad_left : pad_left + w] = x
    out = np.zeros((n, oh_n, ow_n, co))
    for kh in range(kh_n):
        for kw in range(kw_n):
            rows = xp[:, kh * dh : kh * dh + sh * oh_n : sh]
            tap = rows[:, :, kw * dw : kw * dw + sw * ow_n : sw]
            out += tap[:, :oh_n, :ow_n] @ f[kh, kw]
    return out


def conv_slice(source_dim, result_index, result_dim, kernel_dim, pad_before, stride, dilation):
    """(load_start, load_size, pad_before, pad_after) of one spatial axis of a
    load_conv2d tile, as lib/xt/XTToNova.cpp:110-142 computes it."""
    result_start = result_index * result_dim
    field = (result_dim - 1) * stride + dilation * (kernel_dim - 1) + 1
    ideal_start = result_start * stride - pad_before
    ideal_end = ideal_start + field
    load_start = max(ideal_start, 0)
    conv_pad_before = load_start - ideal_start
    load_end = min(load_start + (field - conv_pad_before), source_dim)
    return load_start, load_end - load_start, conv_pad_before, ideal_end - load_end


def conv_out_dim(size, kernel, pad_before, pad_after, stride, dilation):
    eff = dilation * (kernel - 1) + 1
    num = size + pad_before + pad_after - eff
    if num < 0:
        raise ValueError("kernel larger than padded input")
    return num // stride + 1
