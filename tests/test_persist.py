"""The on-disk format's helpers (kiv_amd/persist.py), on the CPU: section
headers and tensor payloads round-trip bit for bit in every stored dtype,
and malformed sections are refused with a clear error."""

from __future__ import annotations

import io
import struct

import pytest
import torch

from kiv_amd import persist


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_tensor_round_trip_bit_exact(dtype):
    g = torch.Generator().manual_seed(3)
    t = (torch.randn(2, 3, 5, 8, generator=g) * 100).to(dtype)
    t[0, 0, 0, :4] = torch.tensor([float("inf"), float("-inf"), -0.0, float("nan")], dtype=dtype)
    f = io.BytesIO()
    persist.write_tensor(f, t)
    persist.write_tensor(f, t[:, :, 1:3])  # a non-contiguous view is written in C order
    assert f.tell() == (t.numel() + t[:, :, 1:3].numel()) * t.element_size()
    f.seek(0)
    a = persist.read_tensor(f, tuple(t.shape), dtype, "cpu")
    b = persist.read_tensor(f, (2, 3, 2, 8), dtype, "cpu")
    bits = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}[dtype]
    assert torch.equal(a.view(bits), t.view(bits))
    assert torch.equal(b.view(bits), t[:, :, 1:3].contiguous().view(bits))


def test_payload_is_little_endian_c_order():
    t = torch.tensor([[1.0, 2.0], [3.0, -4.0]], dtype=torch.float32)
    f = io.BytesIO()
    persist.write_tensor(f, t)
    assert f.getvalue() == struct.pack("<4f", 1.0, 2.0, 3.0, -4.0)


def test_header_round_trip_and_errors():
    f = io.BytesIO()
    persist.write_header(f, persist.COLD_MAGIC, {"version": persist.VERSION, "cold_length": 7, "dtype": "bfloat16"})
    raw = f.getvalue()
    assert raw[:8] == b"KIVCOLD1" and struct.unpack("<Q", raw[8:16])[0] == len(raw) - 16
    h = persist.read_header(io.BytesIO(raw), persist.COLD_MAGIC)
    assert h["cold_length"] == 7 and persist.dtype_of(h["dtype"]) == torch.bfloat16
    with pytest.raises(ValueError, match="not a KIVCACH1 section"):
        persist.read_header(io.BytesIO(raw), persist.CACHE_MAGIC)
    with pytest.raises(ValueError, match="truncated"):
        persist.read_header(io.BytesIO(raw[:20]), persist.COLD_MAGIC)
    g = io.BytesIO()
    persist.write_header(g, persist.COLD_MAGIC, {"version": 99})
    with pytest.raises(ValueError, match="unsupported format version"):
        persist.read_header(io.BytesIO(g.getvalue()), persist.COLD_MAGIC)
    with pytest.raises(ValueError, match="truncated payload"):
        persist.read_tensor(io.BytesIO(b"\0" * 6), (2, 2), torch.float16, "cpu")
    with pytest.raises(ValueError, match="unknown stored dtype"):
        persist.dtype_of("int8")
