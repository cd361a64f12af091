"""Pins of the oracle's sampler (oracle/jit_oracle.c, jo_sample_rows and its helpers) against
what fixes each piece independently: Threefry-2x32-20's published known-answer vectors, float64
log-sum-exp, a numpy restatement of mlx_lm's filter chain written from its specification (top-p on
the ascending cumulative mass, top-k as the k largest by (value desc, index asc)), the categorical
draw as searchsorted on a float64 cdf, and the draw frequencies over a grid of uniforms.  The
reference holds no sampler vectors (its tests compare live MLX draws, Q36T/metal/test_sampler.py)."""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from jitengine_amd import sampler as host_sampler
from tests.helpers import bf16_to_f32, f32_to_bf16, sampler_logits

V_SMALL = 4096


# ----------------------------------------------------------------------------- threefry
def test_threefry_known_answers():
    """Random123's kat_vectors for threefry2x32_20 (counter, key -> output)."""
    kat = [((0, 0), (0, 0), (0x6B200159, 0x99BA4EFE)),
           ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
           ((0x243F6A88, 0x85A308D3), (0x13198A2E, 0x03707344), (0xC4923A9C, 0x483DF7A0))]
    for ctr, key, want in kat:
        assert oracle.threefry2x32(key, ctr) == want
        x, y = host_sampler.threefry2x32(key, np.array([ctr[0]], np.uint32), np.array([ctr[1]], np.uint32))
        assert (int(x[0]), int(y[0])) == want


def test_threefry_host_and_oracle_agree():
    rng = np.random.default_rng(3)
    for _ in range(20):
        key = rng.integers(0, 2**32, 2, dtype=np.uint64).astype(np.uint32)
        c = rng.integers(0, 2**32, (2, 64), dtype=np.uint64).astype(np.uint32)
        x, y = host_sampler.threefry2x32(key, c[0], c[1])
        for j in range(0, 64, 7):
            assert oracle.threefry2x32(key, (c[0, j], c[1, j])) == (int(x[j]), int(y[j]))


def test_uniform_from_key():
    rng = np.random.default_rng(4)
    keys = rng.integers(0, 2**32, (500, 2), dtype=np.uint64).astype(np.uint32)
    u = oracle.threefry_uniform(keys)
    for b in range(0, 500, 37):
        y0 = oracle.threefry2x32(keys[b], (0, 0))[0]
        assert u[b] == np.float32(min(np.float32(y0) / np.float32(2.0**32), np.float32(1 - 2**-24)))
    assert np.all((u >= 0) & (u < 1))
    assert abs(float(u.mean()) - 0.5) < 0.05


def test_split_layout():
    """mx.random.split's words: counter (j, j + num) feeds words j and j + num."""
    key = host_sampler.key_from_seed((7 << 32) | 9)
    assert list(key) == [7, 9]
    ks = host_sampler.split(key, 3)
    for j in range(3):
        x, y = oracle.threefry2x32(key, (j, j + 3))
        flat = ks.reshape(-1)
        assert flat[j] == x and flat[j + 3] == y


# ----------------------------------------------------------------------------- ln, lse, lp
def test_log_ge1_close_to_log():
    s = np.concatenate([np.geomspace(1.0, 2.0**21, 20001), 1 + np.arange(1, 200) * 2.0**-23,
                        [1.0, 2.0, 4.0, 248320.0]]).astype(np.float32)
    worst = 0.0
    for v in s:
        got = oracle.log_ge1(float(v))
        want = math.log(float(v))
        worst = max(worst, abs(got - want) / max(want, 2.0**-20))
    assert worst < 4 * 2.0**-24, worst
    assert oracle.log_ge1(1.0) == 0.0


def _lse64(x_u16: np.ndarray) -> np.ndarray:
    x = bf16_to_f32(x_u16).astype(np.float64)
    m = x.max(axis=1, keepdims=True)
    return (m + np.log(np.exp(x - m).sum(axis=1, keepdims=True)))[:, 0]


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5, 7])
def test_logprobs_match_float64_lse(kind):
    """lp = bf16(x - bf16(lse)): the oracle's lse is float64 lse rounded to bf16 wherever that
    value is not within 2^-14 bf16 ulps of a rounding tie."""
    x = sampler_logits(kind, 6, V_SMALL, 40 + kind, scale=4.0)
    lp = oracle.logprobs_rows(x)
    lse = _lse64(x)
    checked = 0
    for b in range(x.shape[0]):
        lb = bf16_to_f32(f32_to_bf16(np.array([lse[b]], np.float32)))[0]
        ulp = 2.0 ** (math.floor(math.log2(abs(lse[b]))) - 7) if lse[b] != 0 else 2.0**-133
        frac = (lse[b] / ulp) % 1.0
        if abs(frac - 0.5) < 2**-14:
            continue
        want = f32_to_bf16((bf16_to_f32(x[b]) - np.float32(lb)).astype(np.float32))
        assert np.array_equal(lp[b], want), b
        checked += 1
    assert checked >= 4


def test_greedy_is_first_max_of_lp_not_of_logits():
    """Two logits 0 and 2^-8 apart round to one lp when lse ~ 12: the greedy draw takes the
    first index of the largest lp (mx.argmax of the log-probabilities), not the logits' argmax."""
    V = 248320
    x = np.full((1, V), -0.5, np.float32)
    x[0, 10], x[0, 20] = 0.0, 2.0**-8
    xb = f32_to_bf16(x)
    lp = bf16_to_f32(oracle.logprobs_rows(xb))[0]
    assert lp[10] == lp[20] == lp.max()
    assert oracle.argmax_rows(xb)[0] == 10
    assert int(np.argmax(bf16_to_f32(xb)[0])) == 20
    rng = np.random.default_rng(5)
    for kind in (0, 1, 2, 6):
        xb = sampler_logits(kind, 4, V_SMALL, 50 + kind, scale=3.0)
        lp = bf16_to_f32(oracle.logprobs_rows(xb))
        assert np.array_equal(oracle.argmax_rows(xb), np.argmax(lp, axis=1))
    del rng


# ----------------------------------------------------------------------------- filters + draw
def _np_kept(lp: np.ndarray, top_p: float, k: int) -> np.ndarray:
    """mlx_lm's filters written from their specification: apply_top_p keeps the tokens whose
    ascending inclusive cumulative mass (of the bf16 exponentials, rounded to bf16) exceeds
    bf16(1 - top_p), ties in index order; apply_top_k keeps, of those, the k largest by (value
    desc, index asc).  Returns the kept mask in vocabulary order."""
    V = lp.size
    keep = np.ones(V, bool)
    if 0 < top_p < 1:
        thr = float(bf16_to_f32(f32_to_bf16(np.array([1 - top_p], np.float32)))[0])
        order = np.lexsort((np.arange(V), lp))       # ascending value, then index
        uniq, inv = np.unique(lp, return_inverse=True)
        e_u = np.array([oracle.exp_neg(float(v)) for v in uniq], np.float32)
        e = bf16_to_f32(f32_to_bf16(e_u))[inv].astype(np.float64)
        cum = np.cumsum(e[order])
        cum_b = bf16_to_f32(f32_to_bf16(cum.astype(np.float32)))  # exact sums to 2^-42: no double rounding here
        keep[order] = cum_b > thr
        if not keep.any():
            return None
    if 0 < k < V:
        surv = np.flatnonzero(keep)
        if surv.size > k:
            rank = np.lexsort((surv, -lp[surv]))      # value desc, index asc
            keep[:] = False
            keep[surv[rank[:k]]] = True
    return keep


SETTINGS = [(0.7, 0.95, 40), (1.0, 0.9, 20), (0.6, 0.8, 64), (1.3, 1.0, 5), (0.3, 1.0, 0), (1.0, 0.5, 0),
            (1.0, 1.0, 1), (0.7, 0.95, V_SMALL - 1), (0.9, 0.99, 1000)]


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5, 6, 7])
def test_kept_set_and_weights_match_specification(kind):
    x = sampler_logits(kind, 3, V_SMALL, 60 + kind, scale=6.0)
    lp = bf16_to_f32(oracle.logprobs_rows(x))
    for T, p, k in SETTINGS:
        tok, W = oracle.sample_rows(x, T, p, k, np.full(3, 0.5, np.float32), weights=True)
        for b in range(3):
            keep = _np_kept(lp[b], p, k)
            if keep is None:      # nothing survives top-p: the greedy token
                assert not W[b].any() and tok[b] == np.argmax(lp[b])
                continue
            # weights: e^(x - m), x = bf16(lp / T), within 2 fp32 ulps plus the 2^-42 truncation;
            # a kept token's weight is 0 only when e^(x - m) < 2^-42
            assert not np.any((W[b] > 0) & ~keep), (kind, T, p, k, b)
            it = float(bf16_to_f32(f32_to_bf16(np.array([1.0 / T], np.float32)))[0])
            xs = bf16_to_f32(f32_to_bf16((lp[b][keep] * np.float32(it)).astype(np.float32))).astype(np.float64)
            w = np.exp(xs - xs.max())
            got = W[b][keep].astype(np.float64) * 2.0**-42
            assert np.all(np.abs(got - w) <= w * 2.0**-22 + 2.0**-42), (kind, T, p, k, b)
            assert np.all(got[w >= 2.0**-41] > 0)


@pytest.mark.parametrize("kind", [0, 1, 4, 6])
def test_draw_is_the_inverse_cdf(kind):
    """token = searchsorted(cdf, u * sum(w), "right") - 1 on a float64 cdf, except within 1e-9 of
    a boundary; over a grid of N uniforms each token is drawn N w_i / sum(w) times, +-1."""
    x = sampler_logits(kind, 2, 512, 70 + kind, scale=2.0)
    N = 2048
    grid = ((np.arange(N) + 0.5) / N).astype(np.float32)
    for T, p, k in [(1.0, 0.9, 20), (0.7, 1.0, 0), (1.3, 0.95, 64)]:
        for b in range(2):
            toks = oracle.sample_rows(np.repeat(x[b:b + 1], N, axis=0), T, p, k, grid)
            _, W = oracle.sample_rows(x[b:b + 1], T, p, k, grid[:1], weights=True)
            w = W[0].astype(np.float64)
            cdf = np.concatenate([[0.0], np.cumsum(w)[:-1]])
            tot = w.sum()
            ref = np.searchsorted(cdf, grid.astype(np.float64) * tot, side="right") - 1
            near = np.min(np.abs(cdf[None, :] - (grid.astype(np.float64) * tot)[:, None]), axis=1) < 1e-9 * tot
            assert np.array_equal(toks[~near], ref[~near])
            counts = np.bincount(toks, minlength=x.shape[1])
            assert np.all(np.abs(counts - N * w / tot) <= 1.0 + 1e-9)


def test_tiny_rows_exhaustive():
    """All rows of 6 logits from {-1, 0, 1} (729 rows): kept sets for every k and four top_p."""
    import itertools
    rows = np.array(list(itertools.product([-1.0, 0.0, 1.0], repeat=6)), np.float32)
    x = f32_to_bf16(rows)
    lp = bf16_to_f32(oracle.logprobs_rows(x))
    for p in (0.3, 0.5, 0.9, 1.0):
        for k in range(0, 7):
            _, W = oracle.sample_rows(x, 1.0, p, k, np.full(rows.shape[0], 0.25, np.float32), weights=True)
            for b in range(rows.shape[0]):
                keep = _np_kept(lp[b], p, k)
                if keep is None:
                    assert not W[b].any()
                else:
                    assert np.array_equal(W[b] > 0, keep), (b, p, k)


def test_uniform_edges():
    x = sampler_logits(0, 1, V_SMALL, 80)
    u = np.array([0.0, -1.0, np.nan, 1.0, 2.0, 1 - 2**-24], np.float32)
    toks = oracle.sample_rows(np.repeat(x, u.size, axis=0), 1.0, 1.0, 0, u)
    assert toks[0] == toks[1] == toks[2]                  # clamped to 0
    assert toks[3] == toks[4] == toks[5]                  # clamped to 1 - 2^-24
    _, W = oracle.sample_rows(x, 1.0, 1.0, 0, u[:1], weights=True)
    assert toks[0] == np.flatnonzero(W[0])[0]
    assert toks[5] == np.flatnonzero(W[0])[-1]
