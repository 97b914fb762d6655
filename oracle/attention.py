"""CPU oracle for the attention forward -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or as the
timed CPU baseline; the shipped path (``fa_amd``) never imports it and has no
CPU fallback.

What it restates (the reference's algorithm for this path):
  * the op semantics of the reference backend ``npu_fa``
    (``backends/npu_fa/backend.py:36-49``): BNSD layout, non-causal, no mask,
    no dropout, ``scale = dim ** -0.5``, native GQA with query head ``h``
    reading key/value head ``h // (Hq / Hkv)``;
  * the canonical formula ``ref_flash_attn``
    (``backends/expert_v2/impl.py:701-716``): repeat K/V per query group,
    ``softmax(q k^T * scale) v`` computed in FP32, output rounded to FP16;
  * the check of ``core/runner.py:57-72`` / ``core/bench.py:131-144``:
    compare ``out.float()`` with ``ref.float()`` and report ``max|diff|``.

Functions and what pins each (tests/test_oracle.py):
  attention_loops      pure-Python definition for tiny shapes; pinned by
                       hand-computed closed forms (single key, equal logits).
  attention_f64        float64 numpy; pinned against attention_loops, against
                       torch's scaled_dot_product_attention in float64 (the
                       library routine the reference's formula calls), and by
                       closed forms (constant V, identical keys, one dominant
                       key, Nk = 1) and invariants (joint K/V permutation,
                       q shifted orthogonally to every key, GQA == repeated
                       MHA, scale folded into q).
  attention_rows_f64   rows of attention_f64 for sampled (b, h, i); pinned by
                       equality with the full computation (rows are independent).
  attention_f32        the canonical FP32 formula on CPU torch, chunked; pinned
                       against attention_f64 (FP32 rounding bound) and torch's
                       float32 scaled_dot_product_attention. It is also the
                       CPU baseline bench.py times.
  lse_f64 / lse_rows_f64
                       per-row log-sum-exp ln sum_j exp(scale q.k_j), the
                       statistic the kernels' running max and sum encode
                       (the reference keeps them per row in workspace,
                       K32/vector_output.h:22-38, and exports none); pinned by
                       closed forms (one key, identical keys), torch.logsumexp
                       in float64, and the identity attention_f64 ==
                       sum_j exp(scale s_j - lse) v_j.
  block_stats_f64      exact per-key-block statistics the capture mode's
                       online softmax must reproduce: log-sum-exp and max of
                       the scaled scores over each block and over every key
                       up to the block's end (the quantities behind the
                       reference's per-packet m, l, alpha and row-sum dumps,
                       K32/vector_output.h:22-38); pinned by the last prefix
                       equalling lse_f64, each block equalling lse_f64 of its
                       key slice, and the logaddexp recursion of the prefixes.
  causal masks         every function above takes ``causal`` ("none",
                       "top_left": key j <= i, "bottom_right": j <= i + Nk -
                       Nq; a row that sees no key has O = 0, lse = -inf). The
                       reference runs full attention only (sparse_mode=0,
                       backends/npu_fa/backend.py:48; is_causal=False,
                       backends/expert_v2/impl.py:714), so the masks are
                       additions, pinned against torch's float64
                       scaled_dot_product_attention (is_causal=True for
                       top-left, an explicit boolean mask for bottom-right),
                       the closed form O[row 0] = v[key 0] (top-left), prefix
                       consistency (row i equals full attention over keys
                       0..i) and bottom-right's last row equalling full
                       attention.
Every check above plants a mistake in the oracle (dropped scale, swapped GQA
map, transposed operand) and confirms at least one check fails
(tests/test_oracle.py::test_checks_catch_planted_mistakes).
"""

import numpy as np


def _np(x):
    """numpy view of a torch tensor or array-like (CPU)."""
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.asarray(x)


def _scale(d, scale):
    return float(d) ** -0.5 if scale is None else float(scale)


CAUSAL_MODES = ("none", "top_left", "bottom_right")


def key_limit(rows, nq, nk, causal="none"):
    """Index of the last key each query row in ``rows`` sees (-1: no key).

    ``none`` sees all Nk keys; ``top_left`` keys j <= i (torch's
    scaled_dot_product_attention with is_causal=True); ``bottom_right`` keys
    j <= i + Nk - Nq (the last query row sees every key).
    """
    rows = np.asarray(rows, dtype=np.int64)
    if causal == "none":
        return np.full(rows.shape, nk - 1, dtype=np.int64)
    if causal == "top_left":
        return np.minimum(nk - 1, rows)
    if causal == "bottom_right":
        return np.clip(rows + (nk - nq), -1, nk - 1)
    raise ValueError(f"unknown causal mode {causal!r}")


def _mask(s, lim):
    """Scores ``s`` [rows, Nk] with keys past each row's limit set to -inf."""
    if lim is None:
        return s
    j = np.arange(s.shape[-1])
    return np.where(j[None, :] > np.asarray(lim)[:, None], -np.inf, s)


def attention_loops(q, k, v, scale=None, causal="none"):
    """Definition by loops: o[b,h,i] = sum_j softmax_j(q.k_j * scale) v_j over
    the keys row i sees (all, or those up to ``key_limit``).

    Intended for tiny shapes only (pure Python).
    """
    import math

    q, k, v = (_np(t).astype(np.float64) for t in (q, k, v))
    b_, hq, nq, d = q.shape
    hkv, nk = k.shape[1], k.shape[2]
    group = hq // hkv
    sc = _scale(d, scale)
    out = np.zeros((b_, hq, nq, d))
    for b in range(b_):
        for h in range(hq):
            hk = h // group
            for i in range(nq):
                last = int(key_limit([i], nq, nk, causal)[0])
                if last < 0:
                    continue                     # no key: O = 0
                logits = []
                for j in range(last + 1):
                    dot = 0.0
                    for x in range(d):
                        dot += q[b, h, i, x] * k[b, hk, j, x]
                    logits.append(dot * sc)
                mx = max(logits)
                w = [math.exp(t - mx) for t in logits]
                z = sum(w)
                for x in range(d):
                    acc = 0.0
                    for j in range(last + 1):
                        acc += w[j] * v[b, hk, j, x]
                    out[b, h, i, x] = acc / z
    return out


def _softmax_rows_f64(s):
    """Row softmax; a row of only -inf (no visible key) becomes zeros."""
    mx = s.max(axis=-1, keepdims=True)
    empty = ~np.isfinite(mx)
    s = s - np.where(empty, 0.0, mx)
    np.exp(s, out=s)
    z = s.sum(axis=-1, keepdims=True)
    s /= np.where(empty, 1.0, z)
    return s


def attention_f64(q, k, v, scale=None, chunk_rows=1024, causal="none"):
    """Exact-as-float64 attention over [B,H,N,D]; returns float64 [B,Hq,Nq,D]."""
    q, k, v = (_np(t) for t in (q, k, v))
    b_, hq, nq, d = q.shape
    hkv, nk = k.shape[1], k.shape[2]
    if hq % hkv:
        raise ValueError("heads_q must be a multiple of heads_kv")
    group = hq // hkv
    sc = _scale(d, scale)
    out = np.empty((b_, hq, nq, d), dtype=np.float64)
    for b in range(b_):
        for h in range(hq):
            kf = k[b, h // group].astype(np.float64)
            vf = v[b, h // group].astype(np.float64)
            for r0 in range(0, nq, chunk_rows):
                qf = q[b, h, r0:r0 + chunk_rows].astype(np.float64)
                lim = None if causal == "none" else \
                    key_limit(np.arange(r0, r0 + len(qf)), nq, nk, causal)
                p = _softmax_rows_f64(_mask((qf @ kf.T) * sc, lim))
                out[b, h, r0:r0 + chunk_rows] = p @ vf
    return out


def attention_rows_f64(q, k, v, rows, scale=None, causal="none"):
    """float64 output rows for ``rows = [(b, h, i), ...]``; returns [len(rows), D].

    Every output row depends only on its own query row and the full K/V of
    its key/value head, so sampled rows of an N = 131072 problem are exact
    references for the corresponding rows of a full GPU result.
    """
    q, k, v = (_np(t) for t in (q, k, v))
    hq, nq, d = q.shape[1], q.shape[2], q.shape[3]
    group = hq // k.shape[1]
    sc = _scale(d, scale)
    out = np.empty((len(rows), d), dtype=np.float64)
    by_head = {}
    for n, (b, h, i) in enumerate(rows):
        by_head.setdefault((b, h // group), []).append((n, h, i))
    for (b, hk), items in by_head.items():
        kf = k[b, hk].astype(np.float64)
        vf = v[b, hk].astype(np.float64)
        qf = np.stack([q[b, h, i].astype(np.float64) for _, h, i in items])
        lim = None if causal == "none" else \
            key_limit([i for _, _, i in items], nq, kf.shape[0], causal)
        p = _softmax_rows_f64(_mask((qf @ kf.T) * sc, lim))
        res = p @ vf
        for m, (n, _, _) in enumerate(items):
            out[n] = res[m]
    return out


def _lse_rows(s):
    """ln sum exp over the last axis of float64 scores, max-shifted (-inf for
    a row of only -inf)."""
    mx = s.max(axis=-1)
    safe = np.where(np.isfinite(mx), mx, 0.0)
    with np.errstate(divide="ignore"):
        return safe + np.log(np.exp(s - safe[..., None]).sum(axis=-1))


def lse_f64(q, k, scale=None, chunk_rows=1024, causal="none"):
    """float64 [B, Hq, Nq]: lse[b,h,i] = ln sum_j exp(scale * q[b,h,i] . k[b,h//g,j])."""
    q, k = _np(q), _np(k)
    b_, hq, nq, d = q.shape
    group = hq // k.shape[1]
    sc = _scale(d, scale)
    nk = k.shape[2]
    out = np.empty((b_, hq, nq), dtype=np.float64)
    for b in range(b_):
        for h in range(hq):
            kf = k[b, h // group].astype(np.float64)
            for r0 in range(0, nq, chunk_rows):
                qf = q[b, h, r0:r0 + chunk_rows].astype(np.float64)
                lim = None if causal == "none" else \
                    key_limit(np.arange(r0, r0 + len(qf)), nq, nk, causal)
                out[b, h, r0:r0 + chunk_rows] = _lse_rows(_mask((qf @ kf.T) * sc, lim))
    return out


def lse_rows_f64(q, k, rows, scale=None, causal="none"):
    """float64 log-sum-exp for ``rows = [(b, h, i), ...]`` (rows are independent)."""
    q, k = _np(q), _np(k)
    hq, nq, d = q.shape[1], q.shape[2], q.shape[3]
    group = hq // k.shape[1]
    nk = k.shape[2]
    sc = _scale(d, scale)
    out = np.empty(len(rows), dtype=np.float64)
    for n, (b, h, i) in enumerate(rows):
        s = (k[b, h // group].astype(np.float64) @ q[b, h, i].astype(np.float64)) * sc
        s = _mask(s[None, :], key_limit([i], nq, nk, causal))[0]
        out[n] = _lse_rows(s)
    return out


def block_stats_f64(q, k, block, scale=None, causal="none"):
    """Exact statistics per key block of ``block`` keys (the last may be ragged).

    Returns float64 arrays of shape [nblk, B, Hq, Nq]:
      lse_prefix  ln sum exp(scale s_j) over keys j < min((n+1) * block, Nk)
      lse_block   ln sum exp(scale s_j) over block n's keys
      max_prefix  max scale * s_j over the prefix
      max_block   max scale * s_j over block n
    """
    q, k = _np(q), _np(k)
    b_, hq, nq, d = q.shape
    nk = k.shape[2]
    group = hq // k.shape[1]
    sc = _scale(d, scale)
    nblk = -(-nk // block)
    out = {n: np.empty((nblk, b_, hq, nq)) for n in ("lse_prefix", "lse_block", "max_prefix", "max_block")}
    lim = None if causal == "none" else key_limit(np.arange(nq), nq, nk, causal)
    for b in range(b_):
        for h in range(hq):
            s = (q[b, h].astype(np.float64) @ k[b, h // group].astype(np.float64).T) * sc
            s = _mask(s, lim)
            for n in range(nblk):
                blk = s[:, n * block:(n + 1) * block]
                pre = s[:, :(n + 1) * block]
                out["lse_block"][n, b, h] = _lse_rows(blk)
                out["lse_prefix"][n, b, h] = _lse_rows(pre)
                out["max_block"][n, b, h] = blk.max(axis=-1)
                out["max_prefix"][n, b, h] = pre.max(axis=-1)
    return out


def attention_f32(q, k, v, scale=None, chunk_elems=1 << 26):
    """The canonical FP32 formula on CPU torch: FP16 [B,Hq,Nq,D] result.

    K/V heads are repeated per query group implicitly (query head h reads
    key/value head h // group), scores and softmax run in float32, and the
    output is rounded to FP16, as in the reference's ``ref_flash_attn``.
    """
    import torch

    q, k, v = (t if isinstance(t, torch.Tensor) else torch.from_numpy(np.asarray(t))
               for t in (q, k, v))
    b_, hq, nq, d = q.shape
    hkv, nk = k.shape[1], k.shape[2]
    group = hq // hkv
    sc = _scale(d, scale)
    out = torch.empty((b_, hq, nq, d), dtype=torch.float16)
    rows = max(1, min(group * nq, chunk_elems // max(nk, 1)))
    for b in range(b_):
        for hk in range(hkv):
            kf = k[b, hk].float()
            vf = v[b, hk].float()
            qg = q[b, hk * group:(hk + 1) * group].reshape(group * nq, d)
            og = out[b, hk * group:(hk + 1) * group].view(group * nq, d)
            for r0 in range(0, group * nq, rows):
                s = torch.matmul(qg[r0:r0 + rows].float(), kf.t()) * sc
                og[r0:r0 + rows] = torch.matmul(torch.softmax(s, dim=-1), vf).to(torch.float16)
    return out


def sample_rows(shape, count, seed=1234):
    """``count`` distinct (b, h, i) triples spread over a [B,H,N,D] output.

    Always includes the first and last row of the tensor so both ends of the
    query range are covered.
    """
    b_, h_, n_, _ = shape
    total = b_ * h_ * n_
    rng = np.random.default_rng(seed)
    flat = rng.choice(total, size=min(count, total), replace=False)
    flat = np.unique(np.concatenate([flat, [0, total - 1]]))
    return [(int(f // (h_ * n_)), int((f // n_) % h_), int(f % n_)) for f in flat]


def max_abs_diff(out, ref):
    """``max |out - ref|`` in float64, the reference harness's reported statistic."""
    return float(np.max(np.abs(_np(out).astype(np.float64) - _np(ref).astype(np.float64))))
