"""mc_accept_noalloc (the acceptance that allocates nothing, its state in a per-GPU device
array) against mc_accept on the same inputs, bit for bit: two calls in a row, the second
with fewer rows and drafts, then the size limit and the bad-draft error."""
import ctypes as C

import numpy as np
import pytest

from tests._common import f32_to_bf16

pytestmark = pytest.mark.gpu


class DeviceArrays:
    """Device copies of numpy arrays through the HIP runtime the library itself uses (the test
    allocates; the entry point under test does not)."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so.7")
        self.ptrs = []

    def put(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), C.c_size_t(max(a.nbytes, 4))) == 0
        self.ptrs.append(p)
        assert self.rt.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), 1) == 0  # host to device
        return p.value

    def get(self, ptr: int, like: np.ndarray) -> np.ndarray:
        out = np.empty_like(like)
        assert self.rt.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(out.nbytes), 2) == 0
        return out

    def free(self):
        for p in self.ptrs:
            self.rt.hipFree(p)
        self.ptrs = []


def _case(rng, B, K, V):
    lg = f32_to_bf16((np.round(rng.standard_normal((B, K + 1, V)) * 4) / 4).astype(np.float32))
    nd = rng.integers(0, K + 1, B).astype(np.int32)
    dr = np.zeros((B, max(K, 1)), dtype=np.int32)
    vals = (lg.astype(np.uint32) << 16).view(np.float32)
    for r in range(B):
        for j in range(nd[r]):  # mostly the argmax: long accepted prefixes
            dr[r, j] = int(np.argmax(vals[r, j])) if rng.integers(0, 4) else int(rng.integers(0, V))
    uni = rng.integers(0, 2 ** 32, (B, K + 1, 2), dtype=np.uint64).astype(np.uint32)
    return lg, dr, nd, uni


def _samplings(hip, B):
    kinds = [dict(), dict(temperature=0.8, seed=7), dict(temperature=1.0, top_p=0.9, seed=8),
             dict(temperature=0.7, top_k=20, min_p=0.05, seed=9), dict(presence_penalty=0.5, logit_bias={3: 2.0}),
             dict(temperature=1.2, repetition_penalty=1.3, seed=10, eos=(5,), min_tokens=2)]
    return [hip.make_sampling(**kinds[r % len(kinds)]) for r in range(B)]


def _device_call(hip, lg, dr, nd, sps, ctrs, uni, acceptance):
    B, K1, V = lg.shape
    K = K1 - 1
    d = DeviceArrays()
    try:
        p_lg, p_dr, p_nd = d.put(lg), d.put(dr[:, :max(K, 1)]), d.put(nd)
        p_u = d.put(uni) if uni is not None else None
        out0 = np.full((B, K1), -7, dtype=np.int32)
        z = np.zeros(B, dtype=np.int32)
        p_out, p_ne, p_keep, p_nacc = d.put(out0), d.put(z), d.put(z), d.put(z)
        hip.accept_noalloc(p_lg, V, B, K, p_dr, p_nd, sps, ctrs, p_u, acceptance, p_out, p_ne, p_keep, p_nacc)
        out, ne = d.get(p_out, out0), d.get(p_ne, z)
        keep, nacc = d.get(p_keep, z), d.get(p_nacc, z)
    finally:
        d.free()
    return [out[r, :ne[r]].tolist() for r in range(B)], keep.tolist(), nacc.tolist()


def test_noalloc_matches_accept(hip):
    rng = np.random.default_rng(2)
    V = 151936
    for B, K, use_u in ((12, 8, False), (5, 3, True)):  # the second call is smaller
        lg, dr, nd, uni = _case(rng, B, K, V)
        sps = _samplings(hip, B)
        ctrs = rng.integers(0, 1000, B).tolist()
        got = _device_call(hip, lg, dr, nd, sps, ctrs, uni if use_u else None, 1)
        rows = [lg[r, :nd[r] + 1] for r in range(B)]
        drafts = [dr[r, :nd[r]].tolist() for r in range(B)]
        want = hip.accept(rows, drafts, sps, ctrs, 1, uniforms=[uni[r, :nd[r] + 1] for r in range(B)] if use_u else None)
        assert got == want, (B, K)
        assert max(want[2]) > 0  # some drafts were accepted


def test_noalloc_limits(hip):
    rng = np.random.default_rng(3)
    lg, dr, nd, _ = _case(rng, 65, 2, 64)
    with pytest.raises(hip.HipError, match="at most 64 rows"):
        _device_call(hip, lg, dr, nd, _samplings(hip, 65), [0] * 65, None, 1)
    lg, dr, nd, _ = _case(rng, 4, 2, 64)
    dr[1, 0], nd[1] = 64, 1  # a draft id outside the vocabulary
    with pytest.raises(hip.HipError, match="out of range"):
        _device_call(hip, lg, dr, nd, _samplings(hip, 4), [0] * 4, None, 1)
