"""CPU model of the reference kernels' rounding (test infrastructure).

The reference's two CCE kernels cannot run here (they need an Ascend NPU),
and its tests hold no output fixtures for the stress inputs. This module
restates, row by row, the points at which each of them rounds, so that the
error their algorithms carry on a given input can be estimated beside the
error of this library's kernel (``tests/kernel_model.py``). It is an
estimate, not a pin: the restated order of the FP32 and FP16 sums inside the
reference's reduction trees and the rounding of its fused vector
instructions are not known bit for bit, so nothing here is asserted against
the reference's own outputs (parity unpinned). What the CPU tests pin is the
blocked recurrence (with every rounding off it reproduces the float64
oracle) and that each rounding point is applied.

Both kernels (``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/project/op_kernel``
= K32, ``backends/cce_fa_nqkq_nz_resident_v13_q768_pool_i4_p128/project/op_kernel``
= K16) process keys in packets of 512 and share the matrix-unit side:

* S = q.k accumulated in FP32 and written out rounded to FP16
  (``QuantMode_t::F322F16``, K32 ``panel_kernel.h:128-136``, K16
  ``panel_kernel.h:131,134``);
* the PV partial of a packet, FP16 P times FP16 V accumulated in FP32 and
  written out rounded to FP16 (K32 ``panel_kernel.h:41-44, 182-183``; K16
  ``panel_kernel.h:43``).

``acc="fp32"`` (K32, FP32 O):

* packet row max over the FP16 scores, widened and multiplied by
  SCALE = 0.08838834764831845 in FP32 (``online_softmax.h:202-204``);
  m = max(m_old, that), the first packet copies (``:206-209``);
* s * SCALE in FP32 (``:187-192``), minus m (``:98-105``), natural exp in
  FP32 (``:106-109``);
* the row sum z over the unrounded FP32 P by a halving tree (``:137-180``);
  alpha = exp(m_old - m) (``:166-174``); P rounded to FP16 (``:121-135``);
* l = alpha l + z, the first packet copies (``vector_output.h:27-28``);
* O (FP32) = O alpha (``:53-61``), then + the FP16 partial (``:63``; the first
  packet converts, ``:64``); at the end O / l rounded to FP16 (``:72-80``).

``acc="fp16"`` (K16, FP16 softmax and FP16 O):

* SCALE = 0.08837890625 (the FP16 value, ``online_softmax.h:9``); m in FP16,
  initialised to -65504 (``:21``); the packet row max of the FP16 scores
  times SCALE in FP16 (``:109-111``), m = max(that, m) (``:112-115``);
* s * SCALE + (-m) in one FP16 multiply-add (``:129-143``), FP16 exp
  (``:150-168``), the row sum of the FP16 P by an FP16 halving tree
  (``:36-41, 51-70``);
* z = float(sum), alpha = exp(float(m_old) - float(m)) in FP32, l = alpha l +
  z (``vector_output.h:80-92``), alpha rounded to FP16 for the merge
  (``:107-110``);
* O (FP16) = alpha O + partial in one FP16 multiply-add, the first packet
  copies (``:155-164``); at the end float(O) / l rounded to FP16 (``:169-180``).

Modelling choices where the reference's instruction semantics are not
visible in its source: FP32 and FP16 multiply-adds round once (``fused``),
exp is correctly rounded, the matrix unit's FP32 sums are exact-then-rounded,
and the halving trees pair element i with element i + n/2 of the row.
"""

import numpy as np

PACKET = 512
SCALE32 = np.float32(0.08838834764831845)
SCALE16 = np.float16(0.08837890625)
M16_INIT = -65504.0


def _identity(x):
    return np.asarray(x, dtype=np.float64)


def _r32(x):
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float64)


def _r16(x):
    return np.asarray(x, dtype=np.float64).astype(np.float16).astype(np.float64)


def _tree_sum(x, rnd):
    """Row sums by a halving tree (x[:, :n/2] + x[:, n/2:], ...), each level rounded."""
    x = np.asarray(x, dtype=np.float64)
    while x.shape[1] > 1:
        h = x.shape[1] // 2
        x = rnd(x[:, :h] + x[:, h:2 * h]) if x.shape[1] % 2 == 0 else \
            np.concatenate([rnd(x[:, :h] + x[:, h:2 * h]), x[:, 2 * h:]], axis=1)
    return x[:, 0]


def _packets_fp32(s16, vh, scale, r32, r16):
    nk = s16.shape[1]
    m = l = o = None
    for j in range(nk // PACKET):
        sb = s16[:, j * PACKET:(j + 1) * PACKET]
        vb = vh[j * PACKET:(j + 1) * PACKET]
        mrow = r32(sb.max(1) * scale)
        m_new = mrow if m is None else np.maximum(m, mrow)
        x = r32(r32(sb * scale) - m_new[:, None])
        p = r32(np.exp(x))
        z = _tree_sum(p, r32)
        part = r16(r32(r16(p) @ vb))
        if m is None:
            l, o = z, part
        else:
            a = r32(np.exp(r32(m - m_new)))
            l = r32(a * l + z)
            o = r32(r32(o * a[:, None]) + part)
        m = m_new
    return r16(r32(o / l[:, None]))


def _packets_fp16(s16, vh, scale, r32, r16, fused):
    nk = s16.shape[1]
    m = np.full(s16.shape[0], M16_INIT)
    l = o = None
    for j in range(nk // PACKET):
        sb = s16[:, j * PACKET:(j + 1) * PACKET]
        vb = vh[j * PACKET:(j + 1) * PACKET]
        m_old = m
        m = np.maximum(r16(sb.max(1) * scale), m_old)
        x = r16(sb * scale - m[:, None]) if fused else r16(r16(sb * scale) - m[:, None])
        p = r16(np.exp(x))
        z = _tree_sum(p, r16)
        part = r16(r32(p @ vb))
        if l is None:
            l, o = z, part
        else:
            a = r32(np.exp(r32(m_old - m)))
            l = r32(a * l + z)
            a16 = r16(a)[:, None]
            o = r16(a16 * o + part) if fused else r16(r16(a16 * o) + part)
    return r16(r32(o / l[:, None]))


def reference_rows(q, k, v, rows, acc="fp32", rounding=True, fused=True, scale=None):
    """Modelled reference output for query rows ``rows`` [(b, h, i)] (float64 [R, D]).

    ``rounding=False`` runs the same packets and merges in float64 with the
    exact scale (``scale``, default D**-0.5): the blocked recurrence alone.
    Nk must be a multiple of the 512-key packet, as the reference requires.
    """
    q, k, v = (np.asarray(t.numpy() if hasattr(t, "numpy") else t) for t in (q, k, v))
    hq, d = q.shape[1], q.shape[3]
    hkv, nk = k.shape[1], k.shape[2]
    if nk % PACKET:
        raise ValueError("the reference kernels take Nk in whole 512-key packets")
    group = hq // hkv
    exact = d ** -0.5 if scale is None else scale
    if rounding:
        r32, r16 = _r32, _r16
        sc = np.float64(SCALE32 if acc == "fp32" else SCALE16)
    else:
        r32 = r16 = _identity
        sc = np.float64(exact)
    rows = [tuple(r) for r in rows]
    out = np.zeros((len(rows), d))
    by_head = {}
    for n, (b, h, _) in enumerate(rows):
        by_head.setdefault((b, h // group), []).append(n)
    for (b, hk), idx in by_head.items():
        qr = np.stack([q[rows[n][0], rows[n][1], rows[n][2]] for n in idx]).astype(np.float64)
        kh, vh = k[b, hk].astype(np.float64), v[b, hk].astype(np.float64)
        s16 = r16(r32(qr @ kh.T))
        if acc == "fp32":
            out[idx] = _packets_fp32(s16, vh, sc, r32, r16)
        else:
            out[idx] = _packets_fp16(s16, vh, sc, r32, r16, fused)
    return out
