"""Shared numerical helpers for the parity tests (not collected by pytest)."""
import numpy as np


def conv_f64(x, w, b, stride=(1, 1), dil=(1, 1), pad=(1, 1, 1, 1), groups=1):
    """Textbook cross-correlation in float64 (NCHW input, OIHW weights)."""
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    n, c, h, wd = x.shape
    k, cg, kh, kw = w.shape
    pt, pb, pl, pr = pad
    xp = np.zeros((n, c, h + pt + pb, wd + pl + pr))
    xp[:, :, pt:pt + h, pl:pl + wd] = x
    oh = (h + pt + pb - ((kh - 1) * dil[0] + 1)) // stride[0] + 1
    ow = (wd + pl + pr - ((kw - 1) * dil[1] + 1)) // stride[1] + 1
    out = np.zeros((n, k, oh, ow))
    kpg = k // groups
    for g in range(groups):
        xs = xp[:, g * cg:(g + 1) * cg]
        ws = w[g * kpg:(g + 1) * kpg]
        for i in range(kh):
            for j in range(kw):
                y0, x0 = i * dil[0], j * dil[1]
                patch = xs[:, :, y0:y0 + stride[0] * (oh - 1) + 1:stride[0],
                           x0:x0 + stride[1] * (ow - 1) + 1:stride[1]]
                out[:, g * kpg:(g + 1) * kpg] += np.einsum(
                    "nchw,kc->nkhw", patch, ws[:, :, i, j])
    if b is not None:
        out += b.astype(np.float64)[None, :, None, None]
    return out


def max_rel_err(actual, expected):
    """max |a - e| / max |e| (normwise relative error)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def assert_close(actual, expected, rtol, what=""):
    """Elementwise |a - e| <= rtol*|e| + rtol*rms(e).

    The reference's comparator is |a - e| <= atol + rtol*|e|
    (test/Numerical/support/numerical_test_support.cpp:701-770); the absolute
    term here is scaled to the data so that outputs that cancel to near zero
    are judged against the size of the tensor, not against zero.
    """
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    atol = rtol * max(float(np.sqrt(np.mean(e ** 2))), 1e-30)
    err = np.abs(a - e)
    bad = err > rtol * np.abs(e) + atol
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} outside rtol {rtol}; max err "
        f"{err.max():.3e}, max |e| {np.abs(e).max():.3e}, normwise {max_rel_err(a, e):.3e}")
