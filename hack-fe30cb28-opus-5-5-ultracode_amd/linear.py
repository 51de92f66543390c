"""The step's GEMMs: frozen NF4 projections forward (Y = X W^T [+ bias]) and backward
(dX = dY W), and the plain fp16 lm_head products (engine.py:1082, 1112, 1163, 1179, 1239, 1293,
1301, 1316, 1376, 1381).

Backend "dequant": the NF4 weight is dequantised by the HIP kernel into an fp16 buffer (bit-exact
with bitsandbytes), then multiplied by hipBLASLt through torch (fp16 in, fp32 accumulate, fp16
out) - the reference's own structure (dequant, then cuBLAS).
"""

import torch

from .ops import NF4Group, dequant

BACKEND = "dequant"


def _weights(w):
    return w.weights if isinstance(w, NF4Group) else [w]


def dequantize(w):
    """fp16 [N, K] of an NF4Weight or NF4Group (one launch for a group)."""
    ws = _weights(w)
    return dequant(ws, ws[0].packed.device)


def nf4_linear(x, w, bias=None):
    """Y = X W^T [+ bias], fp16 [M, N]."""
    wd = dequantize(w)
    if bias is not None:
        return torch.addmm(bias, x, wd.t())
    return x @ wd.t()


def nf4_linear_t(dy, w):
    """dX = dY W, fp16 [M, K]."""
    return dy @ dequantize(w)


def linear(x, w):
    """x W^T for an fp16 weight [V, H] (the lm_head)."""
    return x @ w.t()


def linear_t(g, w):
    """g W for an fp16 weight [V, H]."""
    return g @ w
