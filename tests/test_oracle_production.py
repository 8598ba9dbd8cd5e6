"""The ProductionCache oracle (oracle/production.py) against invariants its
composition must keep: every appended token is in exactly one of the hot tier
and the demoted stream, in order; hot rows are the appended float16 rows bit for
bit; the arenas hold the newest demoted rows, each within half a quantization
step (plus the float16 roundings) of its source row; once over budget every
update ends with exactly ``hot_budget`` hot tokens (one in, the excess out);
and the attention equals a float64 softmax over the same rows."""
import numpy as np
import pytest

from oracle.fp import F16, to_dtype
from oracle.production import ArenaOracle, ProductionCacheOracle


def _rows(rng, H, N, D):
    return to_dtype((rng.standard_normal((H, N, D)) * 1.5).astype(np.float32), F16).astype(np.float32)


def _attn(rng, H, M, N):
    return (rng.integers(0, 64, (1, H, M, N)) / 4096.0).astype(np.float32)


def _run(bits, gs, strategy="importance", steps=60, seed=0):
    """A 64-token prefill with weights, then `steps` one-token updates (weights every
    4th); the state is checked after each decode update.  Returns the oracle and the
    appended K / V rows."""
    rng = np.random.default_rng(seed)
    H, D, budget = 2, 64, 40
    o = ProductionCacheOracle(1, H, D, hot_budget=budget, warm_budget=48, warm_bits=bits, group_size=gs,
                              batch_migration_size=16, protect_initial=2, protect_recent=4, strategy=strategy)
    ks, vs = [], []
    for t in range(-1, steps):
        n_new = 64 if t < 0 else 1
        k, v = _rows(rng, H, n_new, D), _rows(rng, H, n_new, D)
        n_keys = o.hot_k[0].shape[1] + o.warm_k[0].length + n_new
        attn = _attn(rng, H, n_new, n_keys) if t % 4 == 0 or t < 0 else None
        ks.append(k)
        vs.append(v)
        o.update(k, v, 0, attn)
        all_k, all_v = np.concatenate(ks, axis=1), np.concatenate(vs, axis=1)
        if t >= 0:
            _check_state(o, all_k, all_v, budget=budget, step=t)
    return o, all_k, all_v


def _ids(rows_all, rows):
    """Index of each row of `rows` (H, n, D) among the appended rows (head 0)."""
    table = {r.tobytes(): i for i, r in enumerate(rows_all[0])}
    return [table[r.tobytes()] for r in rows[0]]


def _check_state(o, all_k, all_v, budget, step):
    hk, hv = o.hot_k[0], o.hot_v[0]
    hot = _ids(all_k, hk)
    assert hot == sorted(hot), "hot tier out of order"
    np.testing.assert_array_equal(hk, all_k[:, hot])
    np.testing.assert_array_equal(hv, all_v[:, hot])
    demoted = [i for blk in o.demoted_rows[0] for i in _ids(all_k, blk)]
    assert sorted(demoted + hot) == list(range(all_k.shape[1])), "a token was lost or duplicated"
    if step >= 1:
        assert hk.shape[1] == budget
    # the arena holds the newest demoted rows
    w = o.warm_k[0]
    assert w.length + w.dropped == len(demoted)
    if w.length:
        src = all_k[:, demoted[len(demoted) - w.length:]]
        deq = w.dequantize().astype(np.float32)
        gi = np.arange(o.D) // w.gs
        step_sz = w.scales[..., gi]
        # half a step, plus the float16 roundings of (x - min) / scale (up to maxv ulps at 2^-11)
        tol = step_sz * (0.5 + ((1 << w.bits) - 1) * 2.0 ** -10) + np.abs(src) * 2.0 ** -10 + 1e-6
        assert np.all(np.abs(deq - src) <= tol)


@pytest.mark.parametrize("bits,gs", [(4, 64), (2, 32), (8, 64)])
def test_composition_invariants(bits, gs):
    o, _, _ = _run(bits, gs)
    assert o.migrations > 0 and o.warm_k[0].dropped > 0  # the schedule exercises arena overflow


def test_fifo_demotes_oldest_unprotected():
    o, all_k, _ = _run(4, 64, strategy="fifo", steps=10)
    # FIFO takes hot positions [initial, initial + n): after the prefill, tokens 2..17;
    # then the 9 over budget from what is left at positions 2..10 (tokens 18..26), then
    # one per update (tokens 27..35 over the 9 later updates)
    assert _ids(all_k, o.demoted_rows[0][0]) == list(range(2, 18))
    assert _ids(all_k, o.demoted_rows[0][1]) == list(range(18, 27))
    assert [_ids(all_k, b) for b in o.demoted_rows[0][2:]] == [[i] for i in range(27, 36)]
    assert _ids(all_k, o.hot_k[0])[:3] == [0, 1, 36]


def test_attention_matches_float64_softmax():
    o, _, _ = _run(4, 64, steps=12, seed=3)
    rng = np.random.default_rng(9)
    q = rng.standard_normal((2, o.H, 3, o.D)).astype(np.float32)
    got = o.attention(q, 0)
    k, v = o.get_kv(0)
    qf = q.astype(np.float16).astype(np.float64)
    ref = np.zeros(q.shape, np.float64)
    for b in range(2):
        for h in range(o.H):
            for m in range(3):
                s = [float(np.dot(qf[b, h, m], k[h, n].astype(np.float64))) / np.sqrt(o.D) for n in range(k.shape[1])]
                e = np.exp(np.array(s) - max(s))
                ref[b, h, m] = (e / e.sum()) @ v[h].astype(np.float64)
    np.testing.assert_allclose(got, ref, atol=2e-6, rtol=1e-5)


def test_arena_overflow_drops_oldest():
    rng = np.random.default_rng(1)
    a = ArenaOracle(2, 10, 64, 4, 64)
    x = [_rows(rng, 2, n, 64) for n in (4, 4, 4, 10)]
    a.append(x[0])
    a.append(x[1])
    assert a.append(x[2]) == 4 and a.length == 8 and a.dropped == 4  # 8 + 4 > 10: the 4 oldest leave
    ref = ArenaOracle(2, 10, 64, 4, 64)
    ref.append(np.concatenate([x[1], x[2]], axis=1))
    np.testing.assert_array_equal(a.packed, ref.packed)  # per-token quantization: appends compose
    assert a.append(x[3]) == 0 and a.length == 10 and a.dropped == 12  # as large as the arena: emptied first
    with pytest.raises(RuntimeError):
        a.append(_rows(rng, 2, 11, 64))
