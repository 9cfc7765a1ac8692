"""Synthetic inputs and weights for the benchmark configurations.

Each generator is seeded (numpy PCG64) and returns host numpy arrays in the
ncnn layouts: activations [N,C,H,W] (N independent [C,H,W] blobs), conv
weights [K][C][kh][kw], InnerProduct weights [N_out][K].  Distributions follow
the configuration text (uniform inputs, He-normal conv weights, BN folded into
the bias).
"""
from __future__ import annotations

import numpy as np

RESNET18_STAGES = ((64, 56), (128, 28), (256, 14), (512, 7))


def _rng(seed, stream):
    return np.random.default_rng([seed, stream])


def he_normal(rng, shape, fan_in):
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def conv_single(seed=0):
    """Config 1: one 64->64 3x3 s1 p1 conv with bias and fused ReLU on
    1x64x56x56 uniform[-1,1]."""
    r = _rng(seed, 1)
    x = r.uniform(-1, 1, (1, 64, 56, 56)).astype(np.float32)
    w = he_normal(r, (64, 64, 3, 3), 64 * 9)
    b = (r.standard_normal(64) * 0.01).astype(np.float32)
    return x, w, b


def innerproduct(seed=0, m=256, k=2048, n=1000):
    """Config 2: [m,k] uniform[-1,1] x W[n,k] ~ N(0, 1/sqrt(k)) + bias N(0, 0.01)."""
    r = _rng(seed, 2)
    x = r.uniform(-1, 1, (m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = (r.standard_normal(n) * 0.01).astype(np.float32)
    return x, w, b


def resnet_stage(c, hw, n=32, seed=0):
    """Config 3, one stage: input [n,c,hw,hw] uniform[-1,1]; two 3x3 s1 p1
    c->c convs with He-normal weights and BN folded into the bias."""
    r = _rng(seed, 3000 + c)
    x = r.uniform(-1, 1, (n, c, hw, hw)).astype(np.float32)
    w1 = he_normal(r, (c, c, 3, 3), c * 9)
    b1 = (r.standard_normal(c) * 0.01).astype(np.float32)
    w2 = he_normal(r, (c, c, 3, 3), c * 9)
    b2 = (r.standard_normal(c) * 0.01).astype(np.float32)
    return x, w1, b1, w2, b2


def int8_conv(seed=0, n=32, c=128, k=128, hw=28):
    """Config 4 mapped onto the reference's int8 format: integer-valued fp32
    input (input scale 1.0), int8 weights U{-127..127}, per-channel
    s[k] ~ U[1e-4, 1e-2] expressed as weight scale 1/s[k], an int32 bias b[k]
    expressed as the fp32 bias b[k]*s[k], output scale 1.0, term 101 + ReLU."""
    r = _rng(seed, 4)
    x = r.integers(-127, 128, (n, c, hw, hw)).astype(np.float32)
    w = r.integers(-127, 128, (k, c, 3, 3)).astype(np.int8)
    s = r.uniform(1e-4, 1e-2, k).astype(np.float32)
    ws = (np.float32(1.0) / s).astype(np.float32)
    b_i32 = r.integers(-(1 << 15), 1 << 15, k).astype(np.int32)
    bias = (b_i32.astype(np.float32) * s).astype(np.float32)
    return dict(x=x, w=w, ws=ws, bias=bias, input_scale=1.0, output_scale=1.0)


def conv_flops(n, c, k, oh, ow, kh=3, kw=3):
    """Direct-equivalent conv FLOPs 2*N*K*OH*OW*C*kh*kw."""
    return 2.0 * n * k * oh * ow * c * kh * kw


def winograd_flops(n, c, k, oh, ow):
    """Executed Winograd F(4,3) GEMM FLOPs 2*36*T*C*K, T = N*ceil(OH/4)*ceil(OW/4)."""
    t = n * ((oh + 3) // 4) * ((ow + 3) // 4)
    return 2.0 * 36 * t * c * k
