"""Pins the CPU oracle (oracle/attention.py) without trusting its own formula.

Checks: a pure-loop definition, torch's float64 scaled_dot_product_attention
(the library routine the reference's canonical formula calls), closed forms,
invariants, the sampled-row restriction, the FP32 chunked formula, and a test
that plants mistakes in copies of the oracle to show the checks catch them.
"""

import numpy as np
import pytest
import torch

from oracle import attention as orc


def rand_qkv(b, hq, hkv, nq, nk, d, seed=0, sigma=1.0):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((b, hq, nq, d)) * sigma).astype(np.float16)
    k = (rng.standard_normal((b, hkv, nk, d)) * sigma).astype(np.float16)
    v = rng.standard_normal((b, hkv, nk, d)).astype(np.float16)
    return q, k, v


def sdpa_f64(q, k, v, scale=None):
    """torch float64 SDPA with K/V repeated per query group."""
    qt, kt, vt = (torch.from_numpy(np.asarray(t, dtype=np.float64)) for t in (q, k, v))
    g = qt.shape[1] // kt.shape[1]
    kt = kt.repeat_interleave(g, dim=1)
    vt = vt.repeat_interleave(g, dim=1)
    return torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=None, dropout_p=0.0, is_causal=False, scale=scale).numpy()


def test_loops_closed_forms():
    # One key: the output is that key's value row, whatever the logits.
    q, k, v = rand_qkv(1, 2, 1, 3, 1, 4)
    out = orc.attention_loops(q, k, v)
    np.testing.assert_allclose(out, np.broadcast_to(v.astype(np.float64)[:, :1], out.shape))
    # Zero query: equal logits, the output is the mean of the value rows.
    q = np.zeros((1, 1, 2, 4), np.float16)
    _, k, v = rand_qkv(1, 1, 1, 2, 5, 4)
    out = orc.attention_loops(q, k, v)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0].astype(np.float64).mean(0), rtol=1e-12)
    # Two keys, hand-computed: logits a, b -> weights e^a/(e^a+e^b).
    q = np.array([[[[2.0, 0.0]]]], np.float16)
    k = np.array([[[[1.0, 0.0], [0.0, 1.0]]]], np.float16)
    v = np.array([[[[1.0, 0.0], [0.0, 1.0]]]], np.float16)
    out = orc.attention_loops(q, k, v, scale=1.0)
    w = np.exp(2.0) / (np.exp(2.0) + 1.0)
    np.testing.assert_allclose(out[0, 0, 0], [w, 1 - w], rtol=1e-12)


@pytest.mark.parametrize("shape", [(1, 2, 1, 5, 7, 8), (2, 4, 2, 3, 6, 4), (1, 3, 3, 4, 4, 16)])
def test_f64_matches_loops(shape):
    q, k, v = rand_qkv(*shape, seed=3)
    np.testing.assert_allclose(orc.attention_f64(q, k, v), orc.attention_loops(q, k, v),
                               rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("shape,sigma", [((1, 12, 1, 64, 96, 128), 1.0),
                                         ((2, 4, 2, 32, 64, 128), 3.0),
                                         ((1, 8, 8, 16, 40, 64), 1.0)])
def test_f64_matches_torch_sdpa(shape, sigma):
    q, k, v = rand_qkv(*shape, seed=5, sigma=sigma)
    np.testing.assert_allclose(orc.attention_f64(q, k, v), sdpa_f64(q, k, v),
                               rtol=1e-9, atol=1e-11)


def test_f64_closed_forms():
    q, k, v = rand_qkv(1, 12, 1, 64, 128, 128, seed=7)
    # Constant value rows: output equals the constant.
    vc = np.full_like(v, 0.375)
    np.testing.assert_allclose(orc.attention_f64(q, k, vc), 0.375, rtol=1e-12)
    # Identical key rows: uniform softmax, output = mean of the value rows.
    ks = np.broadcast_to(k[:, :, :1], k.shape).copy()
    out = orc.attention_f64(q, ks, v)
    np.testing.assert_allclose(out, np.broadcast_to(v.astype(np.float64).mean(2, keepdims=True),
                                                    out.shape), rtol=1e-9, atol=1e-12)
    # One dominant key: output equals that key's value row.
    kd = np.zeros_like(k)
    qd = np.zeros_like(q)
    qd[..., 0] = 8.0
    kd[:, :, 37, 0] = 64.0          # logit 8*64/sqrt(128) ~ 45 against 0 elsewhere
    out = orc.attention_f64(qd, kd, v)
    np.testing.assert_allclose(out, np.broadcast_to(v[:, :, 37:38].astype(np.float64), out.shape),
                               atol=1e-15)


def test_f64_invariants():
    q, k, v = rand_qkv(2, 6, 2, 32, 80, 128, seed=11)
    ref = orc.attention_f64(q, k, v)
    # Joint permutation of key/value rows.
    perm = np.random.default_rng(0).permutation(80)
    np.testing.assert_allclose(orc.attention_f64(q, k[:, :, perm], v[:, :, perm]), ref,
                               rtol=1e-10, atol=1e-13)
    # GQA equals MHA with repeated K/V heads.
    mha = orc.attention_f64(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1))
    np.testing.assert_allclose(mha, ref, rtol=0, atol=0)
    # The scale can be folded into q.
    np.testing.assert_allclose(orc.attention_f64(q.astype(np.float64) * 0.5, k, v, scale=1.0),
                               orc.attention_f64(q, k, v, scale=0.5), rtol=1e-10, atol=1e-13)


def test_f64_orthogonal_query_shift():
    # Keys live in the first 64 dims; adding anything in the last 64 dims of q
    # leaves every logit, and so the output, unchanged.
    q, k, v = rand_qkv(1, 2, 1, 16, 48, 128, seed=13)
    k[..., 64:] = 0
    q2 = q.copy()
    q2[..., 64:] += np.float16(2.5)
    np.testing.assert_allclose(orc.attention_f64(q2, k, v), orc.attention_f64(q, k, v),
                               rtol=1e-12, atol=1e-14)


def test_rows_match_full():
    q, k, v = rand_qkv(2, 12, 1, 96, 160, 128, seed=17)
    full = orc.attention_f64(q, k, v)
    rows = orc.sample_rows(q.shape, 40, seed=2)
    assert (0, 0, 0) in rows and (1, 11, 95) in rows
    got = orc.attention_rows_f64(q, k, v, rows)
    want = np.stack([full[b, h, i] for b, h, i in rows])
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("shape,sigma", [((1, 12, 1, 128, 256, 128), 1.0),
                                         ((1, 4, 2, 64, 128, 128), 3.0)])
def test_f32_formula(shape, sigma):
    q, k, v = rand_qkv(*shape, seed=19, sigma=sigma)
    got = orc.attention_f32(q, k, v, chunk_elems=1 << 12).float().numpy()
    exact = orc.attention_f64(q, k, v)
    # FP16 output rounding (half an ulp) plus FP32 arithmetic.
    tol = np.abs(exact) * 2.0 ** -11 + 1e-5
    assert np.all(np.abs(got - exact) <= tol)
    qt, kt, vt = (torch.from_numpy(t) for t in (q, k, v))
    g = shape[1] // shape[2]
    sd = torch.nn.functional.scaled_dot_product_attention(
        qt.float(), kt.float().repeat_interleave(g, 1), vt.float().repeat_interleave(g, 1)).half()
    assert orc.max_abs_diff(got, sd) <= 2 ** -10


def test_checks_catch_planted_mistakes():
    """Mutated copies of the f64 oracle must fail at least one of the pinning checks."""
    q, k, v = rand_qkv(1, 4, 2, 8, 12, 16, seed=23)
    truth = orc.attention_loops(q, k, v)
    sd = sdpa_f64(q, k, v)

    def no_scale(q, k, v):
        return orc.attention_f64(q, k, v, scale=1.0)

    def wrong_group_map(q, k, v):          # h % Hkv instead of h // group
        out = np.empty(q.shape)
        for h in range(q.shape[1]):
            out[:, h:h + 1] = orc.attention_f64(q[:, h:h + 1], k[:, h % k.shape[1]:][:, :1],
                                                v[:, h % k.shape[1]:][:, :1])
        return out

    def transposed_v(q, k, v):             # v read as [D, N] instead of [N, D]
        vt = np.ascontiguousarray(np.swapaxes(v[..., :v.shape[2], :v.shape[2]], 2, 3))
        pad = np.zeros_like(v)
        pad[..., :vt.shape[3]] = vt
        return orc.attention_f64(q, k, pad)

    def no_max_subtract(q, k, v):          # exp without max subtraction, then an off-by-one sum
        out = orc.attention_f64(q, k, v)
        return out * (1 + 1e-3)

    for bad in (no_scale, wrong_group_map, transposed_v, no_max_subtract):
        got = bad(q, k, v)
        assert not (np.allclose(got, truth, rtol=1e-9, atol=1e-12)
                    and np.allclose(got, sd, rtol=1e-9, atol=1e-12)), bad.__name__


# --------------------------------------------------------------------------- #
# log-sum-exp
# --------------------------------------------------------------------------- #
def lse_checks(lse_fn, q, k, v):
    """The pinning checks of the LSE oracle; True when every check passes."""
    import torch

    d = q.shape[3]
    sc = d ** -0.5
    group = q.shape[1] // k.shape[1]
    got = lse_fn(q, k)
    # torch.logsumexp in float64, the library routine.
    qt = torch.from_numpy(q.astype(np.float64))
    kt = torch.from_numpy(np.repeat(k, group, axis=1).astype(np.float64))
    ref = torch.logsumexp(qt @ kt.transpose(-1, -2) * sc, dim=-1).numpy()
    ok = np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # Softmax identity: O = sum_j exp(scale s_j - lse) v_j.
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64),
                  np.repeat(k, group, axis=1).astype(np.float64)) * sc
    o = np.einsum("bhij,bhjd->bhid", np.exp(s - got[..., None]),
                  np.repeat(v, group, axis=1).astype(np.float64))
    ok &= np.allclose(o, orc.attention_f64(q, k, v), rtol=1e-10, atol=1e-12)
    return bool(ok)


def test_lse_closed_forms():
    q, k, v = rand_qkv(1, 2, 1, 5, 1, 16, seed=31)
    sc = 16 ** -0.5
    # One key: lse = scale * q . k.
    want = np.einsum("bhid,bjd->bhi", q.astype(np.float64), k[:, 0].astype(np.float64)) * sc
    assert np.allclose(orc.lse_f64(q, k), want, rtol=1e-12, atol=1e-12)
    # Nk identical keys: lse = ln Nk + scale * q . k.
    kk = np.repeat(k, 7, axis=2)
    assert np.allclose(orc.lse_f64(q, kk), want + np.log(7), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shape", [(1, 2, 1, 9, 13, 16), (2, 4, 2, 6, 33, 8)])
def test_lse_against_library_and_identity(shape):
    q, k, v = rand_qkv(*shape, seed=37)
    assert lse_checks(orc.lse_f64, q, k, v)
    rows = [(0, 0, 0), (shape[0] - 1, shape[1] - 1, shape[3] - 1), (0, shape[1] - 1, 2)]
    full = orc.lse_f64(q, k)
    got = orc.lse_rows_f64(q, k, rows)
    assert np.allclose(got, [full[r] for r in rows], rtol=0, atol=1e-12)


def test_lse_checks_catch_planted_mistakes():
    q, k, v = rand_qkv(1, 2, 1, 6, 10, 16, seed=41)

    def log2_base(q, k):                   # log2 instead of ln
        return orc.lse_f64(q, k) / np.log(2)

    def no_scale(q, k):
        return orc.lse_f64(q, k, scale=1.0)

    def max_only(q, k):                    # drops the log of the sum
        s = np.einsum("bhid,bjd->bhij", q.astype(np.float64), k[:, 0].astype(np.float64))
        return s.max(axis=-1) * 16 ** -0.5

    for bad in (log2_base, no_scale, max_only):
        assert not lse_checks(bad, q, k, v), bad.__name__


# --------------------------------------------------------------------------- #
# per-block statistics (capture mode)
# --------------------------------------------------------------------------- #
def block_checks(stats, q, k, block):
    """True when per-block statistics agree with lse_f64 on key slices."""
    nk = k.shape[2]
    ok = np.allclose(stats["lse_prefix"][-1], orc.lse_f64(q, k), rtol=0, atol=1e-10)
    for n in range(stats["lse_block"].shape[0]):
        sl = k[:, :, n * block:min((n + 1) * block, nk)]
        ok &= np.allclose(stats["lse_block"][n], orc.lse_f64(q, sl), rtol=0, atol=1e-10)
        if n:
            ok &= np.allclose(stats["lse_prefix"][n],
                              np.logaddexp(stats["lse_prefix"][n - 1], stats["lse_block"][n]),
                              rtol=0, atol=1e-10)
    ok &= np.allclose(stats["max_prefix"], np.maximum.accumulate(stats["max_block"], axis=0))
    return bool(ok)


@pytest.mark.parametrize("nk,block", [(64, 64), (200, 64), (129, 128), (7, 128)])
def test_block_stats(nk, block):
    q, k, _ = rand_qkv(1, 4, 2, 5, nk, 16, seed=nk)
    st = orc.block_stats_f64(q, k, block)
    assert st["lse_block"].shape == (-(-nk // block), 1, 4, 5)
    assert block_checks(st, q, k, block)


def test_block_stats_catch_planted_mistakes():
    q, k, _ = rand_qkv(1, 2, 1, 4, 200, 16, seed=5)
    good = orc.block_stats_f64(q, k, 64)

    shifted = {n: a.copy() for n, a in good.items()}            # blocks start one key late
    alt = orc.block_stats_f64(q, k[:, :, 1:], 64)
    shifted["lse_block"][:alt["lse_block"].shape[0]] = alt["lse_block"]
    no_scale = orc.block_stats_f64(q, k, 64, scale=1.0)
    swapped = {n: a.copy() for n, a in good.items()}            # prefix and block exchanged
    swapped["lse_prefix"], swapped["lse_block"] = good["lse_block"], good["lse_prefix"]
    for bad in (shifted, no_scale, swapped):
        assert not block_checks(bad, q, k, 64)


# --------------------------------------------------------------------------- #
# causal masks (additions beyond the reference's full attention)
# --------------------------------------------------------------------------- #
def sdpa_causal_f64(q, k, v, causal):
    """torch float64 SDPA under a causal mode: is_causal=True (top-left), or an
    explicit boolean mask tril(diagonal=Nk-Nq) (bottom-right). Rows with no
    visible key come back NaN from torch; they are reported as zeros."""
    qt, kt, vt = (torch.from_numpy(np.asarray(t, dtype=np.float64)) for t in (q, k, v))
    g = qt.shape[1] // kt.shape[1]
    kt, vt = kt.repeat_interleave(g, dim=1), vt.repeat_interleave(g, dim=1)
    sdpa = torch.nn.functional.scaled_dot_product_attention
    if causal == "top_left":
        out = sdpa(qt, kt, vt, is_causal=True)
    else:
        nq, nk = q.shape[2], k.shape[2]
        mask = torch.ones(nq, nk, dtype=torch.bool).tril(diagonal=nk - nq)
        out = sdpa(qt, kt, vt, attn_mask=mask)
    return np.nan_to_num(out.numpy(), nan=0.0)


def causal_checks(attn, q, k, v, causal):
    """True when ``attn(q, k, v)`` passes every pinning check of a causal mode."""
    nq, nk = q.shape[2], k.shape[2]
    group = q.shape[1] // k.shape[1]
    got = attn(q, k, v)
    ok = np.allclose(got, sdpa_causal_f64(q, k, v, causal), rtol=1e-10, atol=1e-12)
    # Prefix consistency: row i is full attention over the keys it sees.
    for i in sorted({0, nq // 2, nq - 1}):
        last = i if causal == "top_left" else i + nk - nq
        last = min(last, nk - 1)
        if last < 0:
            ok &= bool(np.all(got[:, :, i] == 0))
            continue
        full = orc.attention_f64(q[:, :, i:i + 1], k[:, :, :last + 1], v[:, :, :last + 1])
        ok &= np.allclose(got[:, :, i:i + 1], full, rtol=1e-10, atol=1e-12)
    if causal == "top_left":        # row 0 sees key 0 only
        ok &= np.allclose(got[:, :, 0], np.repeat(v[:, :, 0], group, axis=1).astype(np.float64))
    else:                           # the last row sees every key
        ok &= np.allclose(got[:, :, -1], orc.attention_f64(q, k, v)[:, :, -1], rtol=1e-10)
    return bool(ok)


CAUSAL_SHAPES = [(1, 4, 2, 9, 9, 16), (1, 2, 1, 5, 12, 16), (2, 2, 1, 12, 5, 16)]


@pytest.mark.parametrize("shape", CAUSAL_SHAPES)
@pytest.mark.parametrize("causal", ["top_left", "bottom_right"])
def test_causal_f64(shape, causal):
    q, k, v = rand_qkv(*shape, seed=sum(shape))
    assert causal_checks(lambda q, k, v: orc.attention_f64(q, k, v, causal=causal), q, k, v, causal)
    assert np.allclose(orc.attention_loops(q, k, v, causal=causal),
                       orc.attention_f64(q, k, v, causal=causal), rtol=1e-10, atol=1e-12)
    rows = orc.sample_rows(q.shape, 7, seed=3)
    full = orc.attention_f64(q, k, v, causal=causal)
    assert np.allclose(orc.attention_rows_f64(q, k, v, rows, causal=causal),
                       np.stack([full[b, h, i] for b, h, i in rows]), rtol=0, atol=1e-12)


def test_causal_modes_agree_on_square_and_none_is_full():
    q, k, v = rand_qkv(1, 2, 1, 10, 10, 16, seed=8)
    assert np.array_equal(orc.attention_f64(q, k, v, causal="top_left"),
                          orc.attention_f64(q, k, v, causal="bottom_right"))
    assert np.array_equal(orc.attention_f64(q, k, v, causal="none"), orc.attention_f64(q, k, v))
    assert list(orc.key_limit([0, 3, 9], 10, 4, "bottom_right")) == [-1, -1, 3]
    assert list(orc.key_limit([0, 3, 9], 4, 10, "bottom_right")) == [6, 9, 9]
    with pytest.raises(ValueError):
        orc.key_limit([0], 4, 4, "diagonal")


def _masked_f64(q, k, v, limit):
    """Attention with an arbitrary per-row last-key function (planted mistakes)."""
    nq, nk, d = q.shape[2], k.shape[2], q.shape[3]
    group = q.shape[1] // k.shape[1]
    out = np.zeros(q.shape)
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            s = q[b, h].astype(np.float64) @ k[b, h // group].astype(np.float64).T * d ** -0.5
            lim = np.array([limit(i, nq, nk) for i in range(nq)])
            out[b, h] = orc._softmax_rows_f64(orc._mask(s, lim)) @ v[b, h // group].astype(np.float64)
    return out


def test_causal_checks_catch_planted_mistakes():
    q, k, v = rand_qkv(1, 2, 1, 8, 11, 16, seed=13)
    plants = {
        "top_left": [lambda i, nq, nk: i - 1,                  # strict: j < i
                     lambda i, nq, nk: nk - 1,                 # mask ignored
                     lambda i, nq, nk: min(nk - 1, i + nk - nq)],   # bottom-right instead
        "bottom_right": [lambda i, nq, nk: min(nk - 1, i),     # top-left instead
                         lambda i, nq, nk: min(nk - 1, i + nk - nq - 1),   # off by one
                         lambda i, nq, nk: nk - 1 if i % 2 else min(nk - 1, i + nk - nq)],
    }
    for causal, bads in plants.items():
        assert causal_checks(lambda q, k, v: orc.attention_f64(q, k, v, causal=causal), q, k, v, causal)
        for bad in bads:
            assert not causal_checks(lambda q, k, v: _masked_f64(q, k, v, bad), q, k, v, causal)


@pytest.mark.parametrize("causal", ["top_left", "bottom_right"])
def test_causal_lse_and_block_stats(causal):
    q, k, v = rand_qkv(1, 2, 1, 12, 7, 16, seed=17)
    nq, nk = 12, 7
    lse = orc.lse_f64(q, k, causal=causal)
    lim = orc.key_limit(np.arange(nq), nq, nk, causal)
    # torch.logsumexp over the masked float64 scores; no visible key -> -inf.
    s = torch.from_numpy(np.einsum("bhid,bjd->bhij", q.astype(np.float64),
                                   k[:, 0].astype(np.float64)) * 16 ** -0.5)
    s = s.masked_fill(torch.arange(nk)[None, :] > torch.from_numpy(lim)[:, None], float("-inf"))
    assert np.allclose(lse, torch.logsumexp(s, dim=-1).numpy(), rtol=0, atol=1e-12)
    assert np.all(np.isneginf(lse[:, :, lim < 0]))
    # Softmax identity on the rows that see a key.
    o = orc.attention_f64(q, k, v, causal=causal)
    with np.errstate(invalid="ignore"):          # -inf - -inf on rows with no key
        w = np.exp(s.numpy() - lse[..., None])
    w[:, :, lim < 0] = 0
    assert np.allclose(o, np.einsum("bhij,bjd->bhid", w, v[:, 0].astype(np.float64)), atol=1e-12)
    rows = orc.sample_rows(q.shape, 9, seed=2)
    assert np.allclose(orc.lse_rows_f64(q, k, rows, causal=causal),
                       [lse[b, h, i] for b, h, i in rows], rtol=0, atol=1e-12)
    st = orc.block_stats_f64(q, k, 4, causal=causal)
    assert np.allclose(st["lse_prefix"][-1], lse, rtol=0, atol=1e-12)
    for n in range(1, st["lse_block"].shape[0]):
        assert np.allclose(st["lse_prefix"][n], np.logaddexp(st["lse_prefix"][n - 1],
                                                             st["lse_block"][n]), atol=1e-12)
    for n in range(st["lse_block"].shape[0]):     # each block: masked scores of its keys
        blk = s[..., 4 * n:4 * n + 4]
        assert np.allclose(st["lse_block"][n], torch.logsumexp(blk, dim=-1).numpy(), atol=1e-12)
        assert np.allclose(st["max_block"][n], blk.amax(dim=-1).numpy())
