"""The attention parity bar (tests.helpers.assert_attention_parity) can fail: mistakes a paged
decode-attention kernel could make are planted in the CPU oracle's inputs -- one page id pointing
at another sequence's page, a page dropped (its slot repeating the previous page), the last key
left out -- and the bar must reject each result, at short and at BASELINE's 262,144-key context.
Outputs an fp32-accurate kernel would give pass it; one that rounds the probabilities to bf16
before P.V does not (no CPU-only test runs a kernel: the planted results come from the oracle)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.helpers import assert_attention_parity, bf16_to_f32, f32_to_bf16, normal_bf16

SCALE = 128 ** -0.5


def _case(lens, seed, H=32, Hkv=4):
    rng = np.random.default_rng(seed)
    npg = [-(-L // 16) for L in lens]
    total = sum(npg) + 3
    perm = rng.permutation(total)
    table = np.zeros((len(lens), max(npg)), np.int32)
    at = 0
    for i, n in enumerate(npg):
        table[i, :n] = perm[at:at + n]
        at += n
    pool = normal_bf16((total, Hkv, 2, 16 * 128), seed=seed + 1)
    q = normal_bf16((len(lens), H, 128), seed=seed + 2)
    return q, pool, table


def _fp32_kernel(q, pool, table, lens, bf16_p=False):
    """Attention in float32 on the gathered KV (an fp32-accurate kernel); bf16_p rounds every
    probability to bf16 before P.V (one bf16 MFMA operand) while the denominator keeps fp32."""
    B, H, D = q.shape
    Hkv = pool.shape[1]
    G = H // Hkv
    out = np.empty_like(q)
    for b, L in enumerate(lens):
        kc, vc = oracle.kv_gather(pool, table[b], int(L), Hkv, D)
        for kv in range(Hkv):
            qs = bf16_to_f32(q[b, kv * G:(kv + 1) * G])
            s = (qs @ bf16_to_f32(kc[kv]).T) * np.float32(SCALE)
            p = np.exp(s - s.max(1, keepdims=True)).astype(np.float32)
            den = p.sum(1, keepdims=True, dtype=np.float32)
            if bf16_p:
                p = bf16_to_f32(f32_to_bf16(p))
            out[b, kv * G:(kv + 1) * G] = f32_to_bf16((p @ bf16_to_f32(vc[kv])) / den)
    return out


def _reference(q, pool, table, lens):
    cr, exact = oracle.paged_decode_attn(q, pool, table, lens, SCALE, exact=True)
    stock, _ = oracle.sdpa_mlx_f32(q, pool, table, lens, SCALE)
    return cr, exact, stock


LENS = [1, 33, 700, 5000, 40000]


def test_accurate_results_pass_the_bar():
    q, pool, table = _case(LENS, seed=3)
    cr, exact, stock = _reference(q, pool, table, LENS)
    st = assert_attention_parity(cr, exact, stock, what="correctly rounded")
    assert st["min_equal"] == 1.0
    st = assert_attention_parity(_fp32_kernel(q, pool, table, LENS), exact, stock, what="fp32 kernel")
    assert st["min_equal"] >= 0.99


def test_bf16_probabilities_fail_the_bar():
    """One bf16 P per key (each probability rounded by up to 2^-9) moves ~40% of the outputs by an
    ulp: the floor rejects it where the north star's absolute 2e-2 would not."""
    lens = [5000, 40000]
    q, pool, table = _case(lens, seed=4)
    cr, exact, stock = _reference(q, pool, table, lens)
    with pytest.raises(AssertionError):
        assert_attention_parity(_fp32_kernel(q, pool, table, lens, bf16_p=True), exact, stock)


def _mutations(table, lens, b):
    """(name, table, lens) with one mistake in sequence b."""
    L = lens[b]
    j = (L // 16) // 2  # a page in the middle of the sequence
    other = (b + 1) % len(lens)
    wrong = table.copy()
    wrong[b, j] = table[other, 0]
    dropped = table.copy()
    dropped[b, j] = table[b, j - 1]
    short = list(lens)
    short[b] = L - 1
    return [("wrong page", wrong, lens), ("dropped page", dropped, lens), ("last key missing", table, short)]


@pytest.mark.parametrize("b", [2, 4])
def test_planted_mistakes_fail_the_bar(b):
    q, pool, table = _case(LENS, seed=5)
    cr, exact, stock = _reference(q, pool, table, LENS)
    for name, t, ln in _mutations(table, LENS, b):
        bad = oracle.paged_decode_attn(q, pool, t, ln, SCALE)
        with pytest.raises(AssertionError, match=f"sequence {b}"):
            assert_attention_parity(bad, exact, stock, what=name)


def test_planted_mistakes_fail_the_bar_at_262144_keys():
    """BASELINE config 4's context: one 16-key page of 262,144 moves the outputs by about an ulp,
    under the 2e-2 absolute tolerance and the cosine, but not under this bar.  (8 q heads over one
    kv head -- BASELINE's GQA group -- keep the CPU pool at 134 MB.)"""
    lens = [262144, 1000]
    q, pool, table = _case(lens, seed=6, H=8, Hkv=1)
    cr, exact, stock = _reference(q, pool, table, lens)
    assert_attention_parity(cr, exact, stock, what="correctly rounded")
    for name, t, ln in _mutations(table, lens, 0):
        bad = oracle.paged_decode_attn(q, pool, t, ln, SCALE)
        g, w = bf16_to_f32(bad[0]).astype(np.float64), exact[0]
        assert np.abs(g - w).max() < 2e-2  # the north star's absolute bound misses it
        with pytest.raises(AssertionError, match="sequence 0"):
            assert_attention_parity(bad, exact, stock, what=name)
