"""Prefix K/V blocks on the GPU (the reference's prefix cache, TrackA/BlockAwarePrefixCache.swift
and SafetensorsBlockIO.swift, at the device K/V): export of a row's block in the reference's
cache-state layout equals the row's K/V (mc_batch_read_kv) bit for bit; blocks imported into
another row read back the same; a row admitted after a prefix hit (blocks written to
safetensors files, read back, imported, prefill resumed at the matched count) decodes the same
tokens as the row admitted by a full prefill, with the same K/V."""
import numpy as np
import pytest

from mlxcat_amd import prefix_blocks as pb
from tests._common import QWEN3_8B_1L_V4K, TINY, spec

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg", [TINY, QWEN3_8B_1L_V4K], ids=["d64", "d128"])
def test_export_import_match_cache(hip, cfg):
    m = hip.Model(cfg)
    m.init_synthetic(1234)
    b = hip.Batch(m, 3, 900, spec())
    b.fill_synthetic_kv(1, 700, 91)
    L = cfg["n_layers"]
    full = [[b.read_kv(l, 1, w) for w in (0, 1)] for l in range(L)]  # [n_kv][len][d]
    for t0, n in ((0, 256), (256, 256), (512, 188), (3, 61), (699, 1)):
        k, v = b.export_kv_block(1, t0, n)
        for l in range(L):
            assert np.array_equal(k[l], full[l][0][:, t0:t0 + n]), (t0, n, l)
            assert np.array_equal(v[l], full[l][1][:, t0:t0 + n]), (t0, n, l)
    with pytest.raises(hip.HipError):
        b.export_kv_block(1, 600, 101)  # past the row's length
    # blocks in order into another row (an empty one, then over an older, longer K/V)
    for dst in (0, 2):
        if dst == 2:
            b.fill_synthetic_kv(2, 800, 5)
        for t0, n in ((0, 256), (256, 256), (512, 188)):
            k, v = b.export_kv_block(1, t0, n)
            b.import_kv_block(dst, t0, k, v)
            assert b.kv_len(dst) == t0 + n
        for l in range(L):
            for w in (0, 1):
                assert np.array_equal(b.read_kv(l, dst, w), full[l][w]), (dst, l, w)
    with pytest.raises(hip.HipError):
        k, v = b.export_kv_block(1, 0, 10)
        b.import_kv_block(0, 701, k, v)  # a gap after the row's K/V


def _gen(b, row, n_steps):
    out = []
    for _ in range(n_steps):
        t, c, _f = b.step()
        out += t[row, :c[row]].tolist()
    return out


def test_prefix_hit_admission_matches_full_prefill(hip, tmp_path):
    """Row 0 of batch A: full prefill of a 600-token prompt (512- and 87-token chunks).  Its two
    full 256-token blocks go to safetensors files; batch B's row 1 finds them by chain hash,
    imports them and prefills only positions 512-598 (the same chunk A ran), so its first token,
    its decode (greedy and seeded, with proposals) and its K/V equal A's bit for bit."""
    V = TINY["vocab"]
    rng = np.random.default_rng(4)
    head = rng.integers(0, V, 520).tolist()
    prompt = head + head[100:180]  # a repeat: the n-gram proposer has matches
    assert len(prompt) == 600
    m = hip.Model(TINY)
    m.init_synthetic(1234)
    sc = spec(k=4, min_ctx=8, acceptance=1, single_row_only=0, greedy_only=0)
    for kw in (dict(), dict(temperature=0.8, top_p=0.9, seed=77)):
        a = hip.Batch(m, 2, 1024, sc)
        first_a = a.insert(0, prompt, 40, hip.make_sampling(**kw))
        d = tmp_path / ("s" if kw else "g")
        hashes = pb.store_row_blocks(a, 0, prompt, "tiny-synthetic", str(d))
        assert len(hashes) == 2 and all((d / (h.hex() + ".safetensors")).exists() for h in hashes)
        b = hip.Batch(m, 2, 1024, sc)
        b.insert(0, prompt[:50], 40, hip.make_sampling())  # another row in flight
        matched = pb.load_row_prefix(b, 1, prompt, "tiny-synthetic", str(d))
        assert matched == 512 and b.kv_len(1) == 512
        first_b = b.insert_cached(1, prompt, matched, 40, hip.make_sampling(**kw))
        assert first_b == first_a
        assert all(np.array_equal(a.read_kv(l, 0, w), b.read_kv(l, 1, w)) for l in range(TINY["n_layers"])
                   for w in (0, 1))
        assert _gen(a, 0, 6) == _gen(b, 1, 6)
    # a prompt that is exactly two blocks: the last block is given back (one token to prefill)
    b = hip.Batch(m, 2, 1024, sc)
    assert pb.load_row_prefix(b, 0, prompt[:512], "tiny-synthetic", str(tmp_path / "g")) == 256
    with pytest.raises(hip.HipError):
        b.insert_cached(0, prompt[:512], 300, 10, hip.make_sampling())  # the row holds 256
