"""Prefix K/V blocks on disk, in the reference's file format, for rows of a Batch.

The reference's prefix cache (TrackA) cuts a prompt's K/V into chain-hashed blocks of
`block_size` tokens and stores each block as one safetensors file:

- block_hashes: BlockHashing.computeBlockHash / chainHashes (TrackA/BlockHashing.swift:7-58),
  SHA-256 over a canonical byte string that chains each block to the previous block's hash;
- write_block / read_block: SafetensorsBlockIO.snapshot / encode / write / decode
  (TrackA/SafetensorsBlockIO.swift:37-63, 94-127, 129-170, 172-222), tensors
  `layer.<l>.keys` and `layer.<l>.values` of shape [1, n_kv, T, d], format version "4";
- store_row_blocks / load_row_prefix: the reference's storeCache and fetchCache +
  reconstructCache (TrackA/BlockAwarePrefixCache.swift:31-118) over a directory of block
  files, on the device K/V through Batch.export_kv_block / import_kv_block.

The paged block manager, its reference counts, eviction and the SSD tier are not here."""
from __future__ import annotations

import hashlib
import json
import os
import struct
import tempfile

import numpy as np

FORMAT_VERSION = "4"            # SafetensorsBlockIO.swift:35
HASH_FORMAT_VERSION = 1         # BlockHashing.swift:5
MAX_HEADER_BYTES = 16 * 1024 * 1024  # SafetensorsBlockIO.swift:36

_DTYPES = {  # safetensors name -> (numpy dtype, byte width) (SafetensorsBlockIO.swift:224-258,278-289)
    "BOOL": (np.bool_, 1), "U8": (np.uint8, 1), "I8": (np.int8, 1), "U16": (np.uint16, 2), "I16": (np.int16, 2),
    "F16": (np.float16, 2), "BF16": (np.uint16, 2), "U32": (np.uint32, 4), "I32": (np.int32, 4),
    "F32": (np.float32, 4), "U64": (np.uint64, 8), "I64": (np.int64, 8), "F64": (np.float64, 8),
    "C64": (np.complex64, 8),
}


class SafetensorsBlockIOError(Exception):
    """SafetensorsBlockIOError (SafetensorsBlockIO.swift:292-299): kind is one of
    invalidHeader, invalidTensorHeader, invalidTensorOffsets, invalidTensorByteCount."""

    def __init__(self, kind: str, name: str = "", detail: str = ""):
        super().__init__(f"{kind}({name}){': ' + detail if detail else ''}")
        self.kind, self.name = kind, name


def _u32(v: int) -> bytes:
    return struct.pack("<I", v)


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return _u32(len(b)) + b


def block_hash(model_name: str, previous: bytes | None, tokens, block_size: int) -> bytes:
    """computeBlockHash (BlockHashing.swift:7-31): SHA-256 of version byte, the domain string,
    the model name, the block size, the previous hash (length-prefixed, or a zero length),
    the token count and each token as int64, integers little-endian."""
    c = bytearray([HASH_FORMAT_VERSION])
    c += _string("mlxserve-prefix-cache") + _string(model_name) + _u32(block_size)
    c += _u32(len(previous)) + previous if previous is not None else _u32(0)
    toks = [int(t) for t in tokens]
    c += _u32(len(toks)) + struct.pack(f"<{len(toks)}q", *toks)
    return hashlib.sha256(bytes(c)).digest()


def block_hashes(model_name: str, tokens, block_size: int) -> list[bytes]:
    """chainHashes (BlockHashing.swift:33-54): one hash per full block, each chained to the last."""
    toks = list(tokens)
    out, prev = [], None
    for b in range(len(toks) // block_size):
        prev = block_hash(model_name, prev, toks[b * block_size:(b + 1) * block_size], block_size)
        out.append(prev)
    return out


def encode_block(tensors: dict, metadata: dict) -> bytes:
    """encode (SafetensorsBlockIO.swift:94-127): tensors sorted by name, a JSON header with
    sorted keys and the data offsets, space-padded so the data starts 8-byte aligned, after an
    8-byte little-endian header length.  tensors: name -> (dtype name, shape, raw bytes)."""
    header = {"__metadata__": dict(metadata)}
    off = 0
    names = sorted(tensors)
    for n in names:
        dt, shape, raw = tensors[n]
        header[n] = {"dtype": dt, "shape": [int(x) for x in shape], "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    hb = json.dumps(header, sort_keys=True, separators=(",", ":")).encode("utf-8")
    hb += b" " * ((8 - (8 + len(hb)) % 8) % 8)
    return struct.pack("<Q", len(hb)) + hb + b"".join(tensors[n][2] for n in names)


def decode_block(data: bytes):
    """decode + parseHeader (SafetensorsBlockIO.swift:129-222), with the reference's checks:
    header length within the file and 16 MiB, every tensor entry well-formed, offsets inside
    the data, and byte counts equal to shape x width.  Returns (tensors, metadata), tensors
    name -> numpy array (BF16 as its uint16 bits)."""
    if len(data) < 8:
        raise SafetensorsBlockIOError("invalidHeader")
    hlen = struct.unpack("<Q", data[:8])[0]
    if hlen > MAX_HEADER_BYTES or 8 + hlen > len(data):
        raise SafetensorsBlockIOError("invalidHeader")
    try:
        header = json.loads(data[8:8 + hlen].decode("utf-8"))
    except (UnicodeDecodeError, ValueError) as e:
        raise SafetensorsBlockIOError("invalidHeader", detail=str(e)) from None
    if not isinstance(header, dict):
        raise SafetensorsBlockIOError("invalidHeader")
    meta = header.get("__metadata__")
    meta = {k: v for k, v in meta.items() if isinstance(v, str)} if isinstance(meta, dict) else {}
    start = 8 + hlen
    out = {}
    for name, t in header.items():
        if name == "__metadata__":
            continue
        ok = (isinstance(t, dict) and t.get("dtype") in _DTYPES and isinstance(t.get("shape"), list)
              and isinstance(t.get("data_offsets"), list) and len(t["data_offsets"]) == 2
              and all(isinstance(x, int) and x >= 0 for x in t["shape"])
              and all(isinstance(x, int) for x in t["data_offsets"])
              and t["data_offsets"][0] >= 0 and t["data_offsets"][1] >= t["data_offsets"][0])
        if not ok:
            raise SafetensorsBlockIOError("invalidTensorHeader", name)
        a, b = start + t["data_offsets"][0], start + t["data_offsets"][1]
        if b > len(data):
            raise SafetensorsBlockIOError("invalidTensorOffsets", name)
        np_dt, width = _DTYPES[t["dtype"]]
        want = int(np.prod(t["shape"], dtype=np.int64)) * width
        if b - a != want:
            raise SafetensorsBlockIOError("invalidTensorByteCount", name, f"expected {want}, got {b - a}")
        out[name] = np.frombuffer(data[a:b], dtype=np_dt).reshape(t["shape"])
    return out, meta


def block_metadata(block_hash_: bytes, n_layers: int, token_count: int, model_name: str, block_size: int) -> dict:
    """snapshot's metadata (SafetensorsBlockIO.swift:51-61)."""
    return {"formatVersion": FORMAT_VERSION, "blockHash": block_hash_.hex(), "tokenCount": str(token_count),
            "numLayers": str(n_layers), "modelName": model_name, "blockSize": str(block_size), "isRotating": "0"}


def write_block(path: str, keys: np.ndarray, values: np.ndarray, block_hash_: bytes, token_count: int,
                model_name: str, block_size: int) -> None:
    """snapshot + write (SafetensorsBlockIO.swift:37-83): keys / values [n_layers][n_kv][T][d]
    bf16 bits become layer.<l>.keys / .values of shape [1, n_kv, T, d]; the file is written
    to a temporary name in the same directory and moved into place."""
    L = keys.shape[0]
    tensors = {}
    for l in range(L):
        for nm, arr in (("keys", keys[l]), ("values", values[l])):
            a = np.ascontiguousarray(arr, dtype=np.uint16)
            tensors[f"layer.{l}.{nm}"] = ("BF16", (1,) + a.shape, a.tobytes())
    data = encode_block(tensors, block_metadata(block_hash_, L, token_count, model_name, block_size))
    d = os.path.dirname(os.path.abspath(path))
    os.makedirs(d, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix="." + os.path.basename(path) + ".", suffix=".tmp", dir=d)
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(data)
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise


def read_block(path: str):
    """read (SafetensorsBlockIO.swift:85-88): (keys, values, metadata), keys / values
    [n_layers][n_kv][T][d] uint16 from the layer.<l>.keys / .values tensors."""
    with open(path, "rb") as f:
        tensors, meta = decode_block(f.read())
    L = int(meta.get("numLayers", "0"))
    keys, values = [], []
    for l in range(L):
        for nm, acc in (("keys", keys), ("values", values)):
            t = tensors.get(f"layer.{l}.{nm}")
            if t is None:
                raise SafetensorsBlockIOError("missingTensor", f"layer.{l}.{nm}")
            acc.append(t.reshape(t.shape[1:]) if t.ndim == 4 and t.shape[0] == 1 else t)
    return np.stack(keys), np.stack(values), meta


def block_path(directory: str, block_hash_: bytes) -> str:
    return os.path.join(directory, block_hash_.hex() + ".safetensors")


def store_row_blocks(batch, row: int, tokens, model_name: str, directory: str, block_size: int = 256) -> list[bytes]:
    """storeCache (BlockAwarePrefixCache.swift:88-118) for one row: every full block of
    `tokens` whose K/V the row holds is exported from the device and written as
    <hash hex>.safetensors under `directory` (existing files are kept).  Returns the hashes."""
    hashes = block_hashes(model_name, tokens, block_size)
    n_kv = batch.kv_len(row)
    out = []
    for b, h in enumerate(hashes):
        if (b + 1) * block_size > n_kv:
            break
        p = block_path(directory, h)
        if not os.path.exists(p):
            k, v = batch.export_kv_block(row, b * block_size, block_size)
            write_block(p, k, v, h, block_size, model_name, block_size)
        out.append(h)
    return out


def load_row_prefix(batch, row: int, tokens, model_name: str, directory: str, block_size: int = 256) -> int:
    """fetchCache + reconstructCache (BlockAwarePrefixCache.swift:31-85) for one row: the
    longest run of leading blocks of `tokens` found under `directory` is imported into the
    row, block after block; a full-prompt match gives back its last block, so that at least
    one prompt token is left to prefill (Scheduler.swift:898-929).  Returns the matched
    token count (0: no hit, the row untouched), for Batch.insert_cached."""
    hashes = block_hashes(model_name, tokens, block_size)
    found = []
    for h in hashes:
        if not os.path.exists(block_path(directory, h)):
            break
        found.append(h)
    while found and len(found) * block_size >= len(tokens):
        found.pop()
    for b, h in enumerate(found):
        k, v, meta = read_block(block_path(directory, h))
        if meta.get("blockHash") != h.hex() or int(meta.get("blockSize", "0")) != block_size:
            raise SafetensorsBlockIOError("incompatibleMetadata", h.hex())
        batch.import_kv_block(row, b * block_size, k, v)
    return len(found) * block_size
