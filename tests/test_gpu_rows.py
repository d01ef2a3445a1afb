"""Row compaction and extraction of the device K/V (BatchKVCache.filter(keeping:) and
extract(_:), BatchCache.swift:196-246) on the GPU: a filtered batch's rows keep producing,
token for token, what the same rows produce in a batch that was not filtered, with equal K/V;
a row's K/V extracted into another batch and admitted from its history continues the same
way."""
import numpy as np
import pytest

from mlxcat_amd import _lib
from tests._common import TINY, spec

pytestmark = pytest.mark.gpu
R, K, CTX = 8, 4, 256


def _prompt(r, V):
    if r % 3 == 2:
        return [(i * 37 + 11 * r) % V for i in range(40 + 3 * r)]  # no repeats: no proposals
    return [100 + r + i % (5 + r) for i in range(40 + 3 * r)]


def _sampling(hip, r):
    if r % 4 == 1:
        return hip.make_sampling(temperature=0.8, seed=70 + r, presence_penalty=0.5, frequency_penalty=0.2)
    if r % 4 == 3:
        return hip.make_sampling(temperature=0.6, top_p=0.9)  # unseeded: the batch's own stream
    return hip.make_sampling()


def _make(hip, m):
    b = hip.Batch(m, R, CTX, spec(k=K, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0))
    for r in range(R):
        b.insert(r, _prompt(r, TINY["vocab"]), 60, _sampling(hip, r))
    _steps(b, 2)
    return b


def _steps(b, n):
    out = [[] for _ in range(b.R)]
    for _ in range(n):
        t, c, _f = b.step()
        for r in range(b.R):
            out[r] += t[r, :c[r]].tolist()
    return out


def _same_kv(a, ra, b, rb):
    if a.kv_len(ra) != b.kv_len(rb):
        return False
    return all(np.array_equal(a.read_kv(l, ra, w), b.read_kv(l, rb, w)) for l in range(TINY["n_layers"]) for w in (0, 1))


@pytest.fixture(scope="module")
def model(hip):
    m = hip.Model(TINY)
    m.init_synthetic(1234)
    return m


PLANS = {
    "cycle": [2, 0, 1],                    # 0 <- 2 <- 1 <- 0, rows 3..7 dropped
    "reverse": [7, 6, 5, 4, 3, 2, 1, 0],   # four 2-cycles
    "repeated": [4, 4, 1, 5, 3],           # take() with a row listed twice
    "keep-order": [1, 4, 6],               # increasing: no spare
    "empty": [],
}


@pytest.mark.parametrize("name", list(PLANS))
def test_filter_matches_unfiltered(hip, model, name):
    keep = PLANS[name]
    ref, b = _make(hip, model), _make(hip, model)
    assert b.history(0) == ref.history(0)
    b.filter(keep)
    for i, r in enumerate(keep):
        assert _same_kv(b, i, ref, r), (name, i)
        assert b.history(i) == ref.history(r), (name, i)
    for i in range(len(keep), R):
        assert b.kv_len(i) == 0
    want, got = _steps(ref, 4), _steps(b, 4)
    for i in range(R):
        assert got[i] == (want[keep[i]] if i < len(keep) else []), (name, i)
    assert any(len(want[r]) > 4 for r in keep) or not keep  # rows that speculated took part
    for i, r in enumerate(keep):
        assert _same_kv(b, i, ref, r), (name, i)


def test_extract_kv_then_insert_prefilled(hip, model):
    ref = _make(hip, model)
    one = hip.Batch(model, 1, CTX, spec(k=K, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0))
    for r in (0, 4):  # greedy rows with proposals
        ref.extract_kv(r, one, 0)
        assert _same_kv(one, 0, ref, r)
    hist = ref.history(4)
    assert one.kv_len(0) == len(hist) - 1
    one.insert_prefilled(0, hist, 60, _sampling(hip, 4))
    want, got = _steps(ref, 3), _steps(one, 3)
    assert got[0] == want[4] and len(want[4]) > 3


def test_filter_and_extract_errors(hip, model):
    b = _make(hip, model)
    with pytest.raises(_lib.HipError):
        b.filter([R])
    with pytest.raises(_lib.HipError):
        b.filter([-1, 0])
    small = hip.Batch(model, 1, 32, spec(k=K, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0))
    assert b.kv_len(0) > 32
    with pytest.raises(_lib.HipError):
        b.extract_kv(0, small, 0)  # more positions than the destination holds


def test_filter_and_extract_at_unaligned_capacities(hip, model):
    """Capacities that are not multiples of 64: the cache's position stride is the capacity
    rounded up to a 64-key sub-chunk, and rows moved between batches of different strides
    (250 -> 256, 190 -> 192, 170 -> 192) read back the same K/V and keep decoding the same."""
    sc = spec(k=K, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0)
    a = hip.Batch(model, 3, 250, sc)
    for r in range(3):
        a.insert(r, _prompt(r, TINY["vocab"]), 40, _sampling(hip, r))
    _steps(a, 2)
    e = hip.Batch(model, 1, 190, sc)
    a.extract_kv(2, e, 0)
    assert _same_kv(e, 0, a, 2)
    f = hip.Batch(model, 2, 170, sc)
    e.extract_kv(0, f, 1)
    assert _same_kv(f, 1, a, 2)
    b = hip.Batch(model, 3, 250, sc)
    for r in range(3):
        b.insert(r, _prompt(r, TINY["vocab"]), 40, _sampling(hip, r))
    _steps(b, 2)
    b.filter([2, 0])
    assert _same_kv(b, 0, a, 2) and _same_kv(b, 1, a, 0)
    want, got = _steps(a, 3), _steps(b, 3)
    assert got[0] == want[2] and got[1] == want[0]
