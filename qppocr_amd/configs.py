"""The five synthetic workloads (inputs and weights, seeded).

1  conv 3x3 s1 p1, N=1, 32->32, 160x160, bias (folded BN) + ReLU; x U[0,1),
   w N(0, sqrt(2/288)), b N(0, 0.1); seed 0.
2  depthwise + hardswish, N=1, pad k/2: (C64 160^2 k3 s1), (C128 80^2 k3 s2),
   (C256 40^2 k5 s1), (C256 40^2 k5 s2); x N(0,1), w N(0, sqrt(2/k^2)),
   b N(0, 0.1); seed 1.
3  det forward 1x3x640x640 (nets.build_det, seed 2).
4  rec forward 32x3x48x320 (nets.build_rec, seed 3).
5  det at 1536^2 + 128 rec lines of widths {80, 88, ..., 1280}, bucketed to
   multiples of 160, <= 64 lines per batch, CTC masked past w/8 (seed 4):
   pipeline.mixed_page and pipeline.PageRunner.
"""
import math

import numpy as np

from .nets import WeightRng

CFG2_CASES = [  # (C, H=W, k, stride)
    (64, 160, 3, 1),
    (128, 80, 3, 2),
    (256, 40, 5, 1),
    (256, 40, 5, 2),
]


def cfg1(seed=0):
    r = WeightRng(seed)
    x = r.uniform((1, 32, 160, 160))
    w = r.normal((32, 32, 3, 3), math.sqrt(2.0 / 288.0))
    b = r.normal((32,), 0.1)
    return x, w, b


def cfg2(seed=1):
    """List of (x, w, b, k, stride) for the four depthwise cases."""
    r = WeightRng(seed)
    out = []
    for c, hw, k, s in CFG2_CASES:
        x = r.normal((1, c, hw, hw), 1.0)
        w = r.normal((c, 1, k, k), math.sqrt(2.0 / (k * k)))
        b = r.normal((c,), 0.1)
        out.append((x, w, b, k, s))
    return out


def conv_out_hw(h, k, s, p):
    return (h + 2 * p - k) // s + 1


def cfg1_bytes_flops():
    """Compulsory bytes (x, w, b, y once each, fp32) and FLOPs (2 x MACs)."""
    x = 32 * 160 * 160
    w = 32 * 32 * 9
    y = 32 * 160 * 160
    return 4 * (x + w + 32 + y), 2 * 32 * 32 * 9 * 160 * 160


def cfg2_bytes_flops(c, hw, k, s):
    oh = conv_out_hw(hw, k, s, k // 2)
    bytes_ = 4 * (c * hw * hw + c * k * k + c + c * oh * oh)
    return bytes_, 2 * c * k * k * oh * oh
