"""The sampler kernels on MI355X (csrc/sampler.hip) against the oracle's restatement of the
reference's chain (Q36/sampler.py:295-297, 371-374, 451-476): log-probabilities, the greedy draw,
temperature / top-p / top-k draws given uniforms and the Threefry uniforms, all bit for bit, on the
reference's vocabulary (248,320) and its self-check rows (normal, integer ties, all equal, sparse
spikes, confident, spread; Q36/sampler.py:546-604), the settings of its tests
(Q36T/metal/test_sampler.py) and the edges (k = 1, k >= V, top_p near 0, uniforms at 0 and 1,
-inf logits, a vocabulary that is not a multiple of 8)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jitengine_amd import ops
from jitengine_amd import sampler as host_sampler
from tests.helpers import bf16_tensor, f32_to_bf16, sampler_logits, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"
V_REF = 248320


@pytest.mark.parametrize("V", [V_REF, 1001])
def test_logprobs_rows_bit_exact(V):
    for kind in (0, 1, 2, 3, 4, 5, 7):
        x = sampler_logits(kind, 4, V, 100 + kind, scale=8.0)
        got = u16(ops.logprobs_rows(bf16_tensor(x, DEV)))
        assert np.array_equal(got, oracle.logprobs_rows(x)), kind


def test_greedy_first_max_of_lp():
    x = np.full((3, V_REF), -0.5, np.float32)
    x[0, 10], x[0, 20] = 0.0, 2.0**-8       # one lp: the first index wins over the larger logit
    x[1, 7] = 3.0
    x[2, :] = 0.0
    xb = f32_to_bf16(x)
    got = ops.argmax_rows(bf16_tensor(xb, DEV)).cpu().numpy()
    assert list(got) == [10, 7, 0]
    assert np.array_equal(got, oracle.argmax_rows(xb))
    for kind in (0, 1, 3, 6, 7):
        xb = sampler_logits(kind, 8, V_REF, 110 + kind, scale=12.0)
        t = bf16_tensor(xb, DEV)
        want = oracle.argmax_rows(xb)
        assert np.array_equal(ops.argmax_rows(t).cpu().numpy(), want), kind
        assert np.array_equal(ops.sample_rows(t, 0.0, 0.9, 20, None).cpu().numpy(), want), kind


def test_split_rows_and_one_workgroup_rows_agree():
    """Log-probabilities and the greedy draw of up to 64 rows run over slices of each row, one
    workgroup a slice; 65 rows take one workgroup a row.  Both against the oracle, with ties of the
    largest lp in different slices, a row whose numbers sit in the last slice only, an all -inf
    row, one-slice rows and an unaligned vocabulary."""
    def bf(v):
        return f32_to_bf16(np.array([v], np.float32))[0]

    for V in (V_REF, 7007, 2000):
        x = sampler_logits(0, 65, V, 180 + V % 97, scale=3.0).astype(np.uint16)
        ninf = np.uint16(0xFF80)
        x[1, :] = f32_to_bf16(np.full(V, -1.0, np.float32))
        x[1, V // 2], x[1, V - 3] = bf(5.0), bf(5.0)
        x[2, :] = ninf
        x[2, V - 1] = bf(-7.5)
        x[3, :] = ninf
        x[4, :] = f32_to_bf16(np.full(V, -0.5, np.float32))
        x[4, V // 3], x[4, V - 5] = bf(0.0), bf(2.0**-8)
        want_tok = oracle.argmax_rows(x)
        want_lp = oracle.logprobs_rows(x)
        assert list(want_tok[1:5]) == [V // 2, V - 1, 0, V // 3]
        for B in (1, 5, 64, 65):
            t = bf16_tensor(x[:B], DEV)
            assert np.array_equal(ops.argmax_rows(t).cpu().numpy(), want_tok[:B]), (V, B)
            assert np.array_equal(ops.sample_rows(t, 0.0, 1.0, 0, None).cpu().numpy(), want_tok[:B]), (V, B)
            assert np.array_equal(u16(ops.logprobs_rows(t)), want_lp[:B]), (V, B)


SETTINGS = [(0.7, 0.95, 40), (1.0, 0.9, 20), (0.6, 0.8, 64), (1.3, 1.0, 5), (0.3, 1.0, 0), (1.0, 0.95, 0),
            (1.0, 0.8, 0), (0.7, 1.0, 20), (1.0, 1.0, 1), (1.0, 0.5, 1000), (1.0, 0.02, 40), (2.0, 1.0, V_REF),
            (1.0, 0.95, V_REF - 1)]


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5, 6, 7])
def test_sample_rows_bit_exact(kind):
    B = 4
    x = sampler_logits(kind, B, V_REF, 120 + kind, scale=4.0 if kind == 6 else 12.0)
    t = bf16_tensor(x, DEV)
    rng = np.random.default_rng(130 + kind)
    for T, p, k in SETTINGS:
        u = rng.random(B).astype(np.float32)
        u[0] = 0.0 if kind % 2 else np.float32(1 - 2**-24)
        got = ops.sample_rows(t, T, p, k, torch.from_numpy(u).to(DEV)).cpu().numpy()
        want = oracle.sample_rows(x, T, p, k, u)
        assert np.array_equal(got, want), (kind, T, p, k, got, want)


def test_sample_rows_grid_of_uniforms():
    """One confident and one spread row under 64 uniforms each: every draw bit-exact."""
    x = np.concatenate([sampler_logits(4, 1, V_REF, 140), sampler_logits(5, 1, V_REF, 141)])
    u = ((np.arange(64) + 0.5) / 64).astype(np.float32)
    xr = np.repeat(x, 64, axis=0)
    ur = np.tile(u, 2)
    for T, p, k in [(1.0, 0.9, 20), (0.7, 0.95, 0), (1.3, 1.0, 64)]:
        got = ops.sample_rows(bf16_tensor(xr, DEV), T, p, k, torch.from_numpy(ur).to(DEV)).cpu().numpy()
        assert np.array_equal(got, oracle.sample_rows(xr, T, p, k, ur)), (T, p, k)


def test_sample_rows_split_over_slices():
    """Draws of up to 64 rows run their weights and walk over slices of each row: 64 rows whose
    tie groups (integer logits) span every slice, cut inside a tie group by top-k and top-p or not
    cut at all, and uniforms across (0, 1)."""
    for kind in (1, 0):
        x = sampler_logits(kind, 64, V_REF, 190 + kind, scale=3.0)
        u = ((np.arange(64) + 0.5) / 64).astype(np.float32)
        for T, p, k in [(1.0, 0.9, 20), (0.7, 1.0, 5000), (1.0, 0.5, 0), (1.3, 1.0, 0)]:
            got = ops.sample_rows(bf16_tensor(x, DEV), T, p, k, torch.from_numpy(u).to(DEV)).cpu().numpy()
            assert np.array_equal(got, oracle.sample_rows(x, T, p, k, u)), (kind, T, p, k)


def test_workspace_variants_equal_the_static_buffer_and_run_on_two_streams():
    """The _ws entry points (a caller's workspace) give the static buffer's results, and two streams
    sampling at once, each with a workspace of its own, both get the oracle's draws."""
    x1 = sampler_logits(1, 32, V_REF, 201, scale=3.0)
    x2 = sampler_logits(0, 8, V_REF, 202, scale=3.0)
    u1 = ((np.arange(32) + 0.5) / 32).astype(np.float32)
    u2 = ((np.arange(8) + 0.25) / 8).astype(np.float32)
    t1, t2 = bf16_tensor(x1, DEV), bf16_tensor(x2, DEV)
    d1, d2 = torch.from_numpy(u1).to(DEV), torch.from_numpy(u2).to(DEV)
    ws1, ws2 = ops.sampler_workspace(DEV), ops.sampler_workspace(DEV)
    assert torch.equal(ops.logprobs_rows(t1, ws1), ops.logprobs_rows(t1))
    assert torch.equal(ops.argmax_rows(t2, ws2), ops.argmax_rows(t2))
    want1 = oracle.sample_rows(x1, 1.0, 0.9, 20, u1)
    want2 = oracle.sample_rows(x2, 0.8, 1.0, 40, u2)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for rep in range(4):
        with torch.cuda.stream(s1):
            a = ops.sample_rows(t1, 1.0, 0.9, 20, d1, ws1)
        with torch.cuda.stream(s2):
            b = ops.sample_rows(t2, 0.8, 1.0, 40, d2, ws2)
        outs.append((a, b))
    torch.cuda.synchronize()
    for a, b in outs:
        assert np.array_equal(a.cpu().numpy(), want1)
        assert np.array_equal(b.cpu().numpy(), want2)


def test_sample_rows_unaligned_vocabulary():
    for V in (1001, 7, 4096 + 3):
        x = sampler_logits(0, 3, V, V, scale=3.0)
        u = np.array([0.1, 0.5, 0.9], np.float32)
        for T, p, k in [(1.0, 0.9, 5), (0.5, 1.0, 0), (1.0, 0.7, 0)]:
            got = ops.sample_rows(bf16_tensor(x, DEV), T, p, k, torch.from_numpy(u).to(DEV)).cpu().numpy()
            assert np.array_equal(got, oracle.sample_rows(x, T, p, k, u)), (V, T, p, k)


def test_threefry_uniform_bit_exact():
    rng = np.random.default_rng(150)
    keys = rng.integers(0, 2**32, (1000, 2), dtype=np.uint64).astype(np.uint32)
    got = ops.threefry_uniform(torch.from_numpy(keys.view(np.int32)).to(DEV)).cpu().numpy()
    assert np.array_equal(got, oracle.threefry_uniform(keys))


def test_sampler_requests_are_reproducible_and_batch_independent():
    """Requests draw under their own key streams: the same seed gives the same tokens, alone or in
    a batch of rows that share its settings; the draw equals the oracle's given the key's uniform."""
    x = sampler_logits(0, 3, V_REF, 160, scale=2.0)
    t = bf16_tensor(x, DEV)
    smp = [host_sampler.Sampler(0.8, 0.9, 40, seed=7 + i, max_steps=600, vocab=V_REF) for i in range(3)]
    steps = [0, 255, 256 + 17]
    rows = host_sampler.sample_rows(t, smp, steps).cpu().numpy()
    again = [host_sampler.Sampler(0.8, 0.9, 40, seed=7 + i, max_steps=600, vocab=V_REF) for i in range(3)]
    solo = [int(again[i](t[i], steps[i]).item()) for i in range(3)]
    assert list(rows) == solo
    u = oracle.threefry_uniform(np.stack([s.key(st) for s, st in zip(smp, steps)]))
    assert np.array_equal(rows, oracle.sample_rows(x, 0.8, 0.9, 40, u))
    greedy = host_sampler.Sampler(0.0, None, None, None, 4, V_REF)
    assert int(greedy(t[0], 0).item()) == oracle.argmax_rows(x[:1])[0]


def test_sampler_contract():
    x = bf16_tensor(sampler_logits(0, 2, 64, 170), DEV)
    u = torch.zeros(2, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):
        ops.sample_rows(x, 1.0, 0.9, -1, u)
    with pytest.raises(ValueError):
        ops.sample_rows(x, 1.0, 0.9, 5, None)
    with pytest.raises(ValueError):
        ops.sample_rows(x, float("nan"), 0.9, 5, u)
    big = torch.zeros((1, (1 << 19) + 8), dtype=torch.bfloat16, device=DEV)
    from jitengine_amd._lib import UnsupportedShape
    with pytest.raises(UnsupportedShape):
        ops.sample_rows(big, 1.0, 0.9, 5, u[:1])
    assert ops.sample_rows(x[:0], 1.0, 0.9, 5, u[:0]).shape == (0,)
