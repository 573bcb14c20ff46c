"""On-disk format of a cold tier and of a whole tiered cache.

The reference keeps its cold tier in process memory only and loses it on
restart.  Here a store's cold rows can be written out and read back:

    section  = magic (8 bytes) | header length (8 bytes, little endian) |
               header (UTF-8 JSON) | payload
    store    = section "KIVCOLD1": header {format, version, dtype, batch,
               num_kv_heads, head_dim, page_size, cold_length, chunk_tokens};
               payload = for each chunk of up to chunk_tokens cold tokens,
               in order: K then V, each [batch, num_kv_heads, tokens,
               head_dim] in the dtype, C order, little endian
    cache    = section "KIVCACH1": header {format, version, prefill_complete,
               decode_step, layers: [{index, kind, ...}]}; payload = per
               layer in header order: its hot K and V (same layout), then,
               for a layer with a cold tier, that store's section

Only the rows are stored.  Loading evicts them again in order, which
rebuilds the pages, the summaries and the radii bit for bit (a page's
summary depends on its rows alone), so the format does not depend on the
device layout of the arena or of the summaries.
"""

from __future__ import annotations

import json
import struct

import numpy as np
import torch

COLD_MAGIC = b"KIVCOLD1"
CACHE_MAGIC = b"KIVCACH1"
VERSION = 1
CHUNK_TOKENS = 65536

_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
_BITS = {torch.float32: np.int32, torch.float16: np.int16, torch.bfloat16: np.int16}
_VIEW = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}


def dtype_name(dtype: torch.dtype) -> str:
    for name, d in _DTYPES.items():
        if d == dtype:
            return name
    raise TypeError(f"no stored form for dtype {dtype}")


def dtype_of(name: str) -> torch.dtype:
    try:
        return _DTYPES[name]
    except KeyError:
        raise ValueError(f"unknown stored dtype {name!r}") from None


def write_header(f, magic: bytes, header: dict) -> None:
    body = json.dumps(header, sort_keys=True).encode()
    f.write(magic)
    f.write(struct.pack("<Q", len(body)))
    f.write(body)


def read_header(f, magic: bytes) -> dict:
    got = f.read(8)
    if got != magic:
        raise ValueError(f"not a {magic.decode()} section (found {got!r})")
    raw = f.read(8)
    if len(raw) != 8:
        raise ValueError("truncated section header")
    (n,) = struct.unpack("<Q", raw)
    body = f.read(n)
    if len(body) != n:
        raise ValueError("truncated section header")
    header = json.loads(body.decode())
    if header.get("version") != VERSION:
        raise ValueError(f"unsupported format version {header.get('version')!r} (expected {VERSION})")
    return header


def write_tensor(f, t: torch.Tensor) -> None:
    """t's elements in C order as little-endian bytes of its dtype."""
    bits = t.detach().contiguous().view(_VIEW[t.dtype]).cpu().numpy()
    f.write(bits.astype(bits.dtype.newbyteorder("<"), copy=False).tobytes())


def read_tensor(f, shape, dtype: torch.dtype, device) -> torch.Tensor:
    count = int(np.prod(shape)) if len(shape) else 1
    nbytes = count * torch.tensor([], dtype=dtype).element_size()
    raw = f.read(nbytes)
    if len(raw) != nbytes:
        raise ValueError(f"truncated payload: expected {nbytes} bytes, found {len(raw)}")
    bits = np.frombuffer(raw, dtype=np.dtype(_BITS[dtype]).newbyteorder("<")).astype(_BITS[dtype], copy=True)
    return torch.from_numpy(bits).view(dtype).reshape(shape).to(device)
