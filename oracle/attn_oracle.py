"""Dense masked-attention oracle in float64 (numpy).  TEST INFRASTRUCTURE ONLY --
see oracle/__init__.py.

Restates the arithmetic the reference runs through torch's eager flex-attention
path (the reference itself holds no attention arithmetic; its ``FlexSelfAttention``
calls ``torch.nn.attention.flex_attention.flex_attention``):

* ``attention_fwd`` -- torch/_higher_order_ops/flex_attention.py:159-267
  (``_math_attention_inner`` + ``math_attention``): S = (Q K^T) * scale, masked
  entries -inf, fully-masked rows give O = 0 and LSE = -inf, GQA by
  ``repeat_interleave`` of K/V over the query-head group (:228-229).  LSE is
  returned in natural log, as ``flex_attention`` returns it
  (torch/nn/attention/flex_attention.py:1575-1600 multiplies the ln2-space value
  back by ln2).
* ``attention_bwd`` -- torch/_higher_order_ops/flex_attention.py:825-994
  (``sdpa_dense_backward``): P = exp(S - LSE), dV = P^T dO, dP = dO V^T,
  Delta = rowsum(O * dO), dS = P * (dP - Delta) (masked to 0), dQ = dS K * scale,
  dK = dS^T Q * scale, dK/dV summed over each GQA group.

Shapes: q [B,Hq,T,D], k/v [B,Hkv,T,D], mask bool [Bm,T,T] with Bm in {1, B}.
"""
from __future__ import annotations

import numpy as np


def _mask_for(mask: np.ndarray, b: int) -> np.ndarray:
    return mask[b if mask.shape[0] > 1 else 0]


def attention_fwd(q, k, v, mask, scale=None):
    """Returns (o float64 [B,Hq,T,D], lse float64 [B,Hq,T] natural log)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)  # torch/nn/attention/flex_attention.py:1544
    o = np.zeros_like(q)
    lse = np.full((B, Hq, T), -np.inf)
    for b in range(B):
        mb = _mask_for(mask, b)
        any_row = mb.any(axis=1)
        for h in range(Hq):
            s = (q[b, h] @ k[b, h // G].T) * scale
            s = np.where(mb, s, -np.inf)
            mx = np.where(any_row, s.max(axis=1), 0.0)
            p = np.exp(s - mx[:, None])
            l = p.sum(axis=1)
            safe_l = np.where(any_row, l, 1.0)
            o[b, h] = (p / safe_l[:, None]) @ v[b, h // G]
            lse[b, h] = np.where(any_row, mx + np.log(safe_l), -np.inf)
    return o, lse


def attention_bwd(q, k, v, o, do, lse, mask, scale=None):
    """Returns (dq, dk, dv) float64; ``lse`` in natural log as from attention_fwd."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    o = np.asarray(o, dtype=np.float64)
    do = np.asarray(do, dtype=np.float64)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(B):
        mb = _mask_for(mask, b)
        for h in range(Hq):
            hk = h // G
            s = (q[b, h] @ k[b, hk].T) * scale
            row_lse = lse[b, h]
            finite = np.isfinite(row_lse)
            p = np.where(mb & finite[:, None],
                         np.exp(s - np.where(finite, row_lse, 0.0)[:, None]), 0.0)
            dv[b, hk] += p.T @ do[b, h]
            dp = do[b, h] @ v[b, hk].T
            delta = (o[b, h] * do[b, h]).sum(axis=1)
            ds = p * (dp - delta[:, None])
            dq[b, h] = ds @ k[b, hk] * scale
            dk[b, hk] += ds.T @ q[b, h] * scale
    return dq, dk, dv


def useful_pairs(mask: np.ndarray, B: int) -> int:
    """Number of allowed (b, q, kv) pairs: the N_pairs of the useful-FLOP count."""
    if mask.shape[0] == 1:
        return int(mask.sum()) * B
    return int(mask.sum())
