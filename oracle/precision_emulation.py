"""Operand-rounding emulation of the fused forward's matrix products
(test infrastructure, never shipped).

The HIP forward forms four products per 64-token chunk on the matrix cores,
each with fp32 accumulation: C . B^T, the decayed mask W (times q) against x,
C . S (the entering state) and B^T . (decay q x) (the chunk's state update).
This module recomputes the forward with the operands of exactly those four
products rounded as a matrix-core scheme would see them, everything else
(cumsums, exponentials, masks, the state recurrence) in float64, so the
error of a rounding scheme can be measured on the CPU without building it:

* ``fp16`` / ``bf16``         -- one product per contraction on rounded operands
* ``split16`` / ``splitbf16`` -- each operand as hi + lo (hi = round(v),
                                 lo = round(v - hi)) and three products
                                 hi.hi + hi.lo + lo.hi (the kernels' scheme:
                                 split fp16 in the forward)
* ``fp32``                    -- no rounding (the chunked algorithm itself)
* ``split16_a`` / ``split16_b`` -- two products: only the left (a) or right (b)
                                 operand split, the other rounded to fp16

``mode`` is one scheme for all four products, or a dict naming one per
product (keys ``cb``, ``wx``, ``cs``, ``u``; missing keys take ``split16``),
which measures what each product contributes on its own.

``q_scale`` models the kernels' per-chunk power-of-two scale of q (the
operands of W . x and of the state update carry q 2^-ek, the products are
multiplied back by 2^ek): ``None`` (no scale), ``"sum"`` (ek from the chunk's
q sum alone, which put the sum in [8, 16)) or ``"sum_max"`` (the same, capped
so the largest |q| of the chunk stays below 1; the kernels' rule,
chunk_q_exp in mamba-ascendc_amd/csrc/ssd_device.h).  The state update's
operand takes 2^-ek here; the kernels use 2^-eN with eN >= ek, which is never
larger.

The chunked algorithm is that of ``oracle.ssd_reference.ssd_chunked_core``
(mamba_torch/ssd_reference.py:113-189) in the kernels' arrangement: q folded
into W and into the state update's right operand instead of into x.  Only
``tests/`` import this module.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

MODES = ("fp32", "fp16", "bf16", "split16", "splitbf16", "split16_a", "split16_b")
PRODUCTS = ("cb", "wx", "cs", "u")


def _round(t: torch.Tensor, kind: str) -> torch.Tensor:
    dt = {"fp16": torch.float16, "bf16": torch.bfloat16}[kind]
    return t.to(dt).to(t.dtype)


def _product(eq: str, a: torch.Tensor, b: torch.Tensor, mode: str) -> torch.Tensor:
    if mode == "fp32":
        return torch.einsum(eq, a, b)
    if mode in ("fp16", "bf16"):
        return torch.einsum(eq, _round(a, mode), _round(b, mode))
    base = "bf16" if mode == "splitbf16" else "fp16"
    ah, bh = _round(a, base), _round(b, base)
    al, bl = _round(a - ah, base), _round(b - bh, base)
    if mode == "split16_a":
        return torch.einsum(eq, ah, bh) + torch.einsum(eq, al, bh)
    if mode == "split16_b":
        return torch.einsum(eq, ah, bh) + torch.einsum(eq, ah, bl)
    return torch.einsum(eq, ah, bh) + torch.einsum(eq, ah, bl) + torch.einsum(eq, al, bh)


def _scale_exp(v: torch.Tensor) -> torch.Tensor:
    """Binary exponent e of v = m 2^e with m in [1, 2), clamped to [-126, 126]
    (-1 for v = 0: frexp's exponent of zero is 0)."""
    return (torch.frexp(v.float()).exponent - 1).clamp(-126, 126)


def chunk_q_exponent(qc: torch.Tensor, rule: str) -> torch.Tensor:
    """ek per (..., chunk) of q laid out [..., T] (padded tokens hold 0):
    ``"sum"`` puts the chunk's q sum in [8, 16); ``"sum_max"`` also keeps the
    largest |q| below 1 (largest in [1/2, 1) where that binds)."""
    e = _scale_exp(qc.sum(-1)) - 3
    if rule == "sum_max":
        e = torch.maximum(e, _scale_exp(qc.abs().amax(-1)) + 1)
    elif rule != "sum":
        raise ValueError(f"q_scale rule {rule!r} is not 'sum' or 'sum_max'")
    return e.clamp(min=-126)


def ssd_forward_emulated(x, dt, A, B, C, mode: str, chunk: int = 64, q_scale=None):
    """y [b, l, h, p] and the final state [b, h, p, n] (float32) of the SSD
    forward with softplus(dt), no D / z / initial state, the four matrix
    products' operands rounded per ``mode`` (one scheme, or a dict per
    product), q scaled per ``q_scale`` and float64 everywhere else."""
    per = dict.fromkeys(PRODUCTS, "split16")
    if isinstance(mode, dict):
        if set(mode) - set(PRODUCTS):
            raise ValueError(f"products {sorted(set(mode) - set(PRODUCTS))} are not among {PRODUCTS}")
        per.update(mode)
    else:
        per = dict.fromkeys(PRODUCTS, mode)
    for m in per.values():
        if m not in MODES:
            raise ValueError(f"mode {m!r} is not one of {MODES}")
    b, l, h, p = x.shape
    g, n = B.shape[2], B.shape[3]
    r = h // g
    T = chunk
    x, B, C = x.double(), B.double(), C.double()
    q = F.softplus(dt.double())
    a = A.double()[None, None, :] * q
    k = math.ceil(l / T)
    pad = k * T - l
    if pad:
        x = F.pad(x, (0, 0, 0, 0, 0, pad))
        q = F.pad(q, (0, 0, 0, pad))
        a = F.pad(a, (0, 0, 0, pad))
        B = F.pad(B, (0, 0, 0, 0, 0, pad))
        C = F.pad(C, (0, 0, 0, 0, 0, pad))
    xc = x.reshape(b, k, T, h, p)
    qc = q.reshape(b, k, T, h)
    cs = a.reshape(b, k, T, h).cumsum(2)
    # 2^-ek per (b, k, h): on the q of W and of the state update's operand
    if q_scale is None:
        fk = torch.ones(b, k, h, dtype=torch.float64)
    else:
        fk = torch.pow(2.0, -chunk_q_exponent(qc.permute(0, 1, 3, 2), q_scale).double())
    Bc = B.repeat_interleave(r, dim=2).reshape(b, k, T, h, n)
    Cc = C.repeat_interleave(r, dim=2).reshape(b, k, T, h, n)
    # (1) C_t . B_s and (2) W[t][s] = (C_t . B_s) exp(cs_t - cs_s) q_s (s <= t) against x
    cb = _product("bkthn,bkshn->bkhts", Cc, Bc, per["cb"])
    csh = cs.permute(0, 1, 3, 2)  # [b, k, h, T]
    lower = torch.tril(torch.ones(T, T, dtype=torch.bool))
    w = torch.where(lower, cb * torch.exp(csh[..., :, None] - csh[..., None, :]), torch.zeros((), dtype=cb.dtype))
    w = w * (qc.permute(0, 1, 3, 2) * fk[..., None])[..., None, :]
    y_diag = _product("bkhts,bkshp->bkthp", w, xc, per["wx"]) / fk[:, :, None, :, None]
    # (4) the chunk's state update B^T . (exp(cs_last - cs_t) q_t x_t)
    to_end = torch.exp(cs[:, :, -1:, :] - cs) * qc * fk[:, :, None, :]
    U = _product("bkthn,bkthp->bkhpn", Bc, xc * to_end[..., None], per["u"]) / fk[..., None, None]
    # (3) exp(cs_t) C_t . S with S the state entering the chunk
    S = torch.zeros(b, h, p, n, dtype=torch.float64)
    ys = []
    for kk in range(k):
        y_off = _product("bthn,bhpn->bthp", Cc[:, kk], S, per["cs"]) * torch.exp(cs[:, kk])[..., None]
        ys.append(y_diag[:, kk] + y_off)
        S = torch.exp(cs[:, kk, -1])[..., None, None] * S + U[:, kk]
    y = torch.stack(ys, 1).reshape(b, k * T, h, p)[:, :l]
    return y.float(), S.float()
