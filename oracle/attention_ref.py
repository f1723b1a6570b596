"""numpy / torch-CPU restatement of the reference attention math.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.

Reference anchors
  attention_reference  -> reference src/reference/attention_ref.py:10-45
  attention_backward_f64 -> gradient of that math (the reference's backward
                          raises: src/flash_attention_sm75/ops.py:47-52)
  expand_kv_for_gqa    -> reference src/flash_attention_sm75/ops.py:6-27
  check_correctness    -> reference src/reference/correctness.py:8-37
  flops                -> reference benchmarks/benchmark_attention.py:78-82
"""
from __future__ import annotations

import math

import numpy as np


def default_scale(head_dim: int) -> float:
    """1/sqrt(D), reference attention_ref.py:24-25 and ops.py:79-80."""
    return 1.0 / math.sqrt(head_dim)


def expand_kv_for_gqa(Q: np.ndarray, K: np.ndarray, V: np.ndarray):
    """repeat_interleave of K, V along heads (reference ops.py:6-27).

    Query head h reads KV head h // (Hq // Hkv).
    """
    h_q, h_kv = Q.shape[1], K.shape[1]
    if h_q == h_kv:
        return K, V
    if h_kv == 0 or h_q % h_kv != 0:
        raise RuntimeError(
            f"GQA expansion: Q heads ({h_q}) not divisible by K/V heads ({h_kv})"
        )
    f = h_q // h_kv
    return np.repeat(K, f, axis=1), np.repeat(V, f, axis=1)


def causal_mask(nq: int, nk: int, causal, row0: int = 0, rows: int | None = None):
    """Boolean [rows, nk] mask of the *hidden* keys of query rows row0.., or None.

    causal = False/0: nothing hidden.  True/1 (top-left): key j hidden from
    query i iff j > i -- the reference's triu(diagonal=1) (attention_ref.py:
    34-40) for nq == nk, and torch SDPA's is_causal for nq != nk.  2
    (bottom-right): iff j > i + nk - nq, the queries being the last nq
    positions of the keys' sequence.  Both agree when nq == nk.
    """
    if not causal:
        return None
    if rows is None:
        rows = nq - row0
    diag = nk - nq if int(causal) == 2 else 0
    cols = np.arange(nk)[None, :]
    rws = np.arange(row0, row0 + rows)[:, None]
    return cols > rws + diag


def visible(attn_mask, shape):
    """Explicit boolean mask (True = the key takes part, torch SDPA's boolean
    attn_mask; no reference counterpart) broadcast to ``shape``, or None."""
    if attn_mask is None:
        return None
    return np.broadcast_to(np.asarray(attn_mask, dtype=bool), shape)


def _softmax_rows_f32(S: np.ndarray) -> np.ndarray:
    """torch.softmax(S, dim=-1) in fp32: exp(S - rowmax) / rowsum.

    A row with every key hidden gives 0 (the kernels' l == 0 -> 1/l = 0 rule,
    reference flash_attention_forward.cu:562), not NaN.
    """
    m = S.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, np.float32(0))
    E = np.exp(S - m, dtype=np.float32)
    tot = E.sum(axis=-1, keepdims=True, dtype=np.float32)
    return E / np.where(tot > 0, tot, np.float32(1))


def attention_reference(Q, K, V, causal=False, scale=None, return_f32=False, attn_mask=None):
    """The reference's math path, restated (attention_ref.py:10-45).

    fp16 [B,H,N,D] inputs -> fp32 upcast (:28-30) -> S = Q K^T * scale (:32)
    -> causal triu(diagonal=1) set to -inf (:34-40) -> softmax(dim=-1) (:42)
    -> P V (:43) -> fp16 (:45).  K, V with fewer heads are expanded first, as
    the reference API does before calling the kernel (ops.py:35-36).
    Materialises [B,H,N,N]; use :func:`attention_reference_chunked` for large
    shapes.
    """
    Q = np.asarray(Q)
    K, V = expand_kv_for_gqa(Q, np.asarray(K), np.asarray(V))
    if scale is None:
        scale = default_scale(Q.shape[-1])
    qf = Q.astype(np.float32)
    kf = K.astype(np.float32)
    vf = V.astype(np.float32)
    S = np.matmul(qf, np.swapaxes(kf, -1, -2)) * np.float32(scale)
    mask = causal_mask(Q.shape[-2], K.shape[-2], causal)
    if mask is not None:
        S[..., mask] = -np.inf
    vis = visible(attn_mask, S.shape)
    if vis is not None:
        S[~vis] = -np.inf
    P = _softmax_rows_f32(S)
    O = np.matmul(P, vf)
    return O if return_f32 else O.astype(np.float16)


def attention_reference_chunked(Q, K, V, causal=False, scale=None, rows=512,
                                heads=None, return_f32=False, attn_mask=None):
    """Same math as :func:`attention_reference`, one (b, h, row block) at a time.

    Rows of the softmax are independent, so evaluating [rows, N] blocks of S
    gives the same values as the full [N, N] matrix (up to fp32 summation
    order inside BLAS).  Under a causal mask a row block only evaluates the
    keys up to its last row's diagonal: the keys past it are hidden from
    every row of the block, so they would contribute exp(-inf) = 0 to the
    row sums and to P V.  ``heads`` restricts the computation to a list of
    query-head indices (output has only those heads), which the CPU baseline
    uses to time a bounded sample.
    """
    Q = np.asarray(Q)
    K = np.asarray(K)
    V = np.asarray(V)
    B, Hq, N, D = Q.shape
    Hkv, Nk = K.shape[1], K.shape[2]
    if Hkv == 0 or Hq % Hkv != 0:
        raise RuntimeError(
            f"GQA expansion: Q heads ({Hq}) not divisible by K/V heads ({Hkv})"
        )
    group = Hq // Hkv
    if scale is None:
        scale = default_scale(D)
    hs = list(range(Hq)) if heads is None else list(heads)
    out = np.empty((B, len(hs), N, D), dtype=np.float32 if return_f32 else np.float16)
    sc = np.float32(scale)
    vis = visible(attn_mask, (B, Hq, N, Nk))
    for b in range(B):
        for oi, h in enumerate(hs):
            kf = K[b, h // group].astype(np.float32)
            vf = V[b, h // group].astype(np.float32)
            kt = np.ascontiguousarray(kf.T)
            diag = Nk - N if int(causal) == 2 else 0
            for r0 in range(0, N, rows):
                r1 = min(N, r0 + rows)
                # keys any row of the block can see: j <= (r1 - 1) + diag
                kc = min(Nk, max(0, r1 + diag)) if causal else Nk
                if kc == 0:
                    out[b, oi, r0:r1] = 0
                    continue
                qf = Q[b, h, r0:r1].astype(np.float32)
                S = (qf @ kt[:, :kc]) * sc
                mask = causal_mask(N, Nk, causal, r0, r1 - r0)
                if mask is not None:
                    S[mask[:, :kc]] = -np.inf
                if vis is not None:
                    S[~vis[b, h, r0:r1, :kc]] = -np.inf
                P = _softmax_rows_f32(S)
                o = P @ vf[:kc]
                out[b, oi, r0:r1] = o if return_f32 else o.astype(np.float16)
    return out


def attention_lse(Q, K, causal=False, scale=None, dtype=np.float64, attn_mask=None):
    """Row log-sum-exp: LSE_i = log sum_{j visible} exp(scale * q_i . k_j).

    No reference counterpart (the reference names LSE only as future work);
    this is the closed form the kernel's optional LSE output must equal.
    """
    Q = np.asarray(Q)
    K = np.asarray(K)
    B, Hq, N, D = Q.shape
    group = Hq // K.shape[1]
    if scale is None:
        scale = default_scale(D)
    out = np.empty((B, Hq, N), dtype=dtype)
    vis = visible(attn_mask, (B, Hq, N, K.shape[2]))
    for b in range(B):
        for h in range(Hq):
            q = Q[b, h].astype(dtype)
            k = K[b, h // group].astype(dtype)
            S = (q @ k.T) * dtype(scale)
            mask = causal_mask(N, K.shape[2], causal)
            if mask is not None:
                S[mask] = -np.inf
            if vis is not None:
                S[~vis[b, h]] = -np.inf
            m = S.max(axis=-1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0)
            with np.errstate(divide="ignore"):
                out[b, h] = (m[:, 0] + np.log(np.exp(S - m).sum(axis=-1)))
    return out


def attention_f64(Q, K, V, causal=False, scale=None, attn_mask=None):
    """Brute-force float64 attention (two-pass softmax), for pinning the fp32 path."""
    Q = np.asarray(Q)
    K, V = expand_kv_for_gqa(Q, np.asarray(K), np.asarray(V))
    if scale is None:
        scale = default_scale(Q.shape[-1])
    q = Q.astype(np.float64)
    k = K.astype(np.float64)
    v = V.astype(np.float64)
    S = np.matmul(q, np.swapaxes(k, -1, -2)) * float(scale)
    mask = causal_mask(Q.shape[-2], K.shape[-2], causal)
    if mask is not None:
        S[..., mask] = -np.inf
    vis = visible(attn_mask, S.shape)
    if vis is not None:
        S[~vis] = -np.inf
    m = S.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    E = np.exp(S - m)
    tot = E.sum(axis=-1, keepdims=True)
    return np.matmul(E / np.where(tot > 0, tot, 1.0), v)


def attention_backward_f64(Q, K, V, dO, causal=False, scale=None, attn_mask=None,
                           delta_from_o=None):
    """Gradients (dQ, dK, dV) of attention_f64's O in float64, closed form.

    No reference counterpart: the reference's autograd backward raises
    (ops.py:47-52).  This is the textbook gradient of the math path of
    attention_ref.py:24-45, O = softmax(scale Q K^T + mask) V:
      P = softmax(S), dV = P^T dO, dP = dO V^T,
      dS = P o (dP - rowsum(dP o P)), dQ = scale dS K, dK = scale dS^T Q.
    A KV head shared by a group of query heads gets the sum of the group's
    gradients (the adjoint of the repeat_interleave at ops.py:24-26).  Rows
    that see no key have P = 0 and contribute nothing.  ``attn_mask``: a
    boolean mask (True = visible) broadcastable to [B, Hq, Nq, Nk], as in
    :func:`attention_reference`.

    ``delta_from_o``: an output O [B, Hq, Nq, D] (e.g. the forward's rounded
    one) from which the row term is taken as rowsum(dO o O) instead, the
    form a fused backward evaluates (rowsum(dP o P) = rowsum(dO o O) for the
    exact O).  Everything else stays exact, so this isolates what O's
    rounding does to the gradients, which is large where dP - rowsum
    nearly cancels (rows that see one or two keys of a peaked softmax).
    """
    Q = np.asarray(Q)
    K = np.asarray(K)
    V = np.asarray(V)
    B, Hq, N, D = Q.shape
    Hkv, Nk = K.shape[1], K.shape[2]
    Ke, Ve = expand_kv_for_gqa(Q, K, V)
    if scale is None:
        scale = default_scale(D)
    q = Q.astype(np.float64)
    k = Ke.astype(np.float64)
    v = Ve.astype(np.float64)
    do = np.asarray(dO).astype(np.float64)
    S = np.matmul(q, np.swapaxes(k, -1, -2)) * float(scale)
    mask = causal_mask(N, Nk, causal)
    if mask is not None:
        S[..., mask] = -np.inf
    vis = visible(attn_mask, S.shape)
    if vis is not None:
        S[~vis] = -np.inf
    m = S.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    E = np.exp(S - m)
    tot = E.sum(axis=-1, keepdims=True)
    P = E / np.where(tot > 0, tot, 1.0)
    dv = np.matmul(np.swapaxes(P, -1, -2), do)
    dP = np.matmul(do, np.swapaxes(v, -1, -2))
    if delta_from_o is None:
        delta = (dP * P).sum(axis=-1, keepdims=True)
    else:
        delta = (do * np.asarray(delta_from_o).astype(np.float64)).sum(axis=-1, keepdims=True)
    dS = P * (dP - delta)
    dq = float(scale) * np.matmul(dS, k)
    dk = float(scale) * np.matmul(np.swapaxes(dS, -1, -2), q)
    g = Hq // Hkv
    dk = dk.reshape(B, Hkv, g, Nk, D).sum(axis=2)
    dv = dv.reshape(B, Hkv, g, Nk, D).sum(axis=2)
    return dq, dk, dv


def check_correctness(output, reference, name="", atol=1e-2, rtol=1e-2):
    """Error metrics of reference correctness.py:8-37 (numpy restatement).

    max/mean abs error, max/mean relative error abs/(|ref|+1e-8), and
    allclose semantics |out - ref| <= atol + rtol*|ref| elementwise.
    """
    o = np.asarray(output, dtype=np.float32)
    r = np.asarray(reference, dtype=np.float32)
    if o.shape != r.shape:
        raise ValueError(f"shape mismatch {o.shape} vs {r.shape}")
    abs_err = np.abs(o - r)
    rel_err = abs_err / (np.abs(r) + np.float32(1e-8))
    finite = bool(np.isfinite(o).all())
    is_close = finite and bool(np.all(abs_err <= atol + rtol * np.abs(r)))
    if o.size == 0:
        return {"name": name, "max_abs_err": 0.0, "mean_abs_err": 0.0,
                "max_rel_err": 0.0, "mean_rel_err": 0.0, "allclose": True,
                "atol": atol, "rtol": rtol}
    return {
        "name": name,
        "max_abs_err": float(abs_err.max()),
        "mean_abs_err": float(abs_err.mean()),
        "max_rel_err": float(rel_err.max()),
        "mean_rel_err": float(rel_err.mean()),
        "allclose": is_close,
        "atol": atol,
        "rtol": rtol,
    }


def flops(batch, heads, seq_len, head_dim, causal=False):
    """Algorithmic FLOPs 4*B*H*N^2*D, halved for causal
    (reference benchmarks/benchmark_attention.py:78-82)."""
    f = 4 * batch * heads * seq_len * seq_len * head_dim
    return f // 2 if causal else f


# ---------------------------------------------------------------------------
# torch-CPU restatement: the reference's CPU PyTorch path, used as the timed
# CPU baseline (same ops as attention_ref.py:28-45, evaluated per (b, h) and
# row block so the [N, N] score matrix fits in host memory).
# ---------------------------------------------------------------------------
def attention_reference_torch_cpu(Q, K, V, causal=False, scale=None, rows=2048, heads=None,
                                  return_f32=False, skip_hidden=False):
    """Square (Nq == Nk) attention per (b, h) and row block with torch on the
    CPU.  Defaults: the reference's op order, full [rows, N] score blocks
    masked afterwards, fp16 output (the timed CPU baseline).  return_f32
    keeps the unrounded fp32 result (parity checks hold the kernel to the
    unrounded value); skip_hidden evaluates a causal row block only up to its
    last row's diagonal (the keys past it are hidden from every row of the
    block and add exp(-inf) = 0), which halves the work of a causal check."""
    import torch

    B, Hq, N, D = Q.shape
    Hkv = K.shape[1]
    group = Hq // Hkv
    if scale is None:
        scale = default_scale(D)
    hs = list(range(Hq)) if heads is None else list(heads)
    out = torch.empty((B, len(hs), N, D), dtype=torch.float32 if return_f32 else torch.float16)
    for b in range(B):
        for oi, h in enumerate(hs):
            k_f = K[b, h // group].float()
            v_f = V[b, h // group].float()
            for r0 in range(0, N, rows):
                r1 = min(N, r0 + rows)
                kc = r1 if causal and skip_hidden else N
                q_f = Q[b, h, r0:r1].float()
                S = torch.matmul(q_f, k_f[:kc].transpose(-2, -1)) * scale
                if causal:
                    mask = torch.ones(r1 - r0, kc, dtype=torch.bool).triu(diagonal=1 + r0)
                    S.masked_fill_(mask, float("-inf"))
                P = torch.softmax(S, dim=-1)
                o = torch.matmul(P, v_f[:kc])
                out[b, oi, r0:r1] = o if return_f32 else o.half()
    return out
