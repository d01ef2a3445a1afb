"""The prefix-block file format and block hashes (TrackA/SafetensorsBlockIO.swift,
TrackA/BlockHashing.swift) on the CPU: the reference's own tests' cases (an exact bf16 byte
round trip, a truncated file refused with invalidTensorOffsets), the files read back by the
independent `safetensors` library, and the hash's canonical byte string laid out by hand
from BlockHashing.swift:7-31 (the reference's tests hold no hash values)."""
import hashlib
import struct

import numpy as np
import pytest

from mlxcat_amd import prefix_blocks as pb


def test_hash_canonical_bytes():
    # version 1 | len 21 "mlxserve-prefix-cache" | len 1 "m" | block size 2 | no previous (0)
    # | 2 tokens | 1, 2 as int64 little-endian
    canon = bytes.fromhex(
        "01" + "15000000" + b"mlxserve-prefix-cache".hex() + "01000000" + b"m".hex() + "02000000" + "00000000"
        + "02000000" + "0100000000000000" + "0200000000000000")
    h0 = pb.block_hash("m", None, [1, 2], 2)
    assert h0 == hashlib.sha256(canon).digest()
    # the next block chains the previous hash, length-prefixed (32 bytes)
    canon1 = bytes.fromhex("01" + "15000000" + b"mlxserve-prefix-cache".hex() + "01000000" + b"m".hex()
                           + "02000000" + "20000000") + h0 + bytes.fromhex(
        "02000000" + "ffffffffffffffff" + "0000000001000000")
    assert pb.block_hash("m", h0, [-1, 2 ** 32], 2) == hashlib.sha256(canon1).digest()


def test_chain_hashes():
    toks = list(range(1000, 1000 + 9))
    hs = pb.block_hashes("model-x", toks, 4)
    assert len(hs) == 2  # full blocks only
    assert hs[0] == pb.block_hash("model-x", None, toks[:4], 4)
    assert hs[1] == pb.block_hash("model-x", hs[0], toks[4:8], 4)
    # a change in block 0 changes every later hash; a change in the tail changes none
    alt = [toks[0] + 1] + toks[1:]
    assert all(a != b for a, b in zip(pb.block_hashes("model-x", alt, 4), hs))
    assert pb.block_hashes("model-x", toks[:8] + [7], 4) == hs
    assert pb.block_hashes("model-y", toks, 4)[0] != hs[0]


def test_exact_bf16_round_trip(tmp_path):
    """exactBF16RoundTrip (TrackAPrefixCacheTests.swift:548-590): raw bf16 bits 0x3f80, 0x4000,
    0xbf80 of shape [1, 1, 3, 1] come back byte for byte, isRotating "0"."""
    raw = np.array([0x3F80, 0x4000, 0xBF80], dtype=np.uint16).reshape(1, 1, 3, 1)
    p = str(tmp_path / "byte" / "roundtrip.safetensors")
    pb.write_block(p, raw, raw, bytes([0xAB] * 32), 3, "byte-test", 3)
    k, v, meta = pb.read_block(p)
    assert k.tobytes() == raw.tobytes() and v.tobytes() == raw.tobytes()
    assert meta["isRotating"] == "0" and meta["formatVersion"] == "4" and meta["blockHash"] == "ab" * 32
    assert meta["tokenCount"] == "3" and meta["numLayers"] == "1" and meta["blockSize"] == "3"
    # the independent reader
    torch = pytest.importorskip("torch")
    from safetensors import safe_open
    with safe_open(p, framework="pt") as f:
        assert f.metadata() == meta
        t = f.get_tensor("layer.0.keys")
        assert t.dtype == torch.bfloat16 and list(t.shape) == [1, 1, 3, 1]
        assert t.view(torch.int16).numpy().astype(np.uint16).tobytes() == raw.tobytes()


def test_layout_matches_safetensors_writer(tmp_path):
    """Header (sorted keys, compact JSON, space padding to 8 bytes) and tensor order (by name,
    so layer.10 sorts before layer.2) as encode writes them; the `safetensors` library reads
    every tensor back."""
    rng = np.random.default_rng(0)
    L, nkv, T, d = 11, 2, 4, 8
    k = rng.integers(0, 2 ** 16, (L, nkv, T, d), dtype=np.uint16)
    v = rng.integers(0, 2 ** 16, (L, nkv, T, d), dtype=np.uint16)
    p = str(tmp_path / "b.safetensors")
    pb.write_block(p, k, v, bytes(range(32)), T, "m", T)
    data = open(p, "rb").read()
    hlen = struct.unpack("<Q", data[:8])[0]
    assert (8 + hlen) % 8 == 0
    import json
    header = json.loads(data[8:8 + hlen])
    names = [n for n in header if n != "__metadata__"]
    order = sorted(names, key=lambda n: header[n]["data_offsets"][0])
    assert order == sorted(names) and order[:3] == ["layer.0.keys", "layer.0.values", "layer.1.keys"]
    assert order[2 * 2] == "layer.10.keys"
    assert data[8:8 + hlen].rstrip(b" ").decode() == json.dumps(header, sort_keys=True, separators=(",", ":"))
    k2, v2, _ = pb.read_block(p)
    assert np.array_equal(k2, k) and np.array_equal(v2, v)
    torch = pytest.importorskip("torch")
    from safetensors.torch import load_file
    t = load_file(p)
    for l in range(L):
        assert t[f"layer.{l}.values"].view(torch.int16).numpy().astype(np.uint16).tobytes() == v[l].tobytes()


def test_truncated_file_is_refused(tmp_path):
    """testSafetensorsReadThrowsOnTruncatedTensorData (TrackAPrefixCacheTests.swift:105-139)."""
    z = np.zeros((1, 1, 2, 2), dtype=np.float32)
    tensors = {f"layer.0.{n}": ("F32", z.shape, z.tobytes()) for n in ("keys", "values")}
    data = pb.encode_block(tensors, pb.block_metadata(bytes([0xCC] * 32), 1, 2, "truncated-test", 2))
    p = tmp_path / "truncated.safetensors"
    p.write_bytes(data[:-1])
    with pytest.raises(pb.SafetensorsBlockIOError) as e:
        pb.read_block(str(p))
    assert e.value.kind == "invalidTensorOffsets"


@pytest.mark.parametrize("mutate,kind", [
    (lambda d: d[:4], "invalidHeader"),
    (lambda d: struct.pack("<Q", 17 * 2 ** 20) + d[8:], "invalidHeader"),
    (lambda d: d.replace(b'"dtype":"F32"', b'"dtype":"F99"', 1), "invalidTensorHeader"),
    (lambda d: d.replace(b'"shape":[1,1,2,2]', b'"shape":[1,1,2,1]', 1), "invalidTensorByteCount"),
])
def test_malformed_headers(tmp_path, mutate, kind):
    z = np.zeros((1, 1, 2, 2), dtype=np.float32)
    data = pb.encode_block({"layer.0.keys": ("F32", z.shape, z.tobytes())}, {"numLayers": "1"})
    p = tmp_path / "bad.safetensors"
    p.write_bytes(mutate(data))
    with pytest.raises(pb.SafetensorsBlockIOError) as e:
        pb.read_block(str(p))
    assert e.value.kind == kind
