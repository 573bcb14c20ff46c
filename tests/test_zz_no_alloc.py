"""kiv_decode_attention_noalloc: the decode attention with its split partials
in the library's static device array instead of a caller workspace.

Called through the C-ABI on two shapes in a row (the second smaller, so a
stale partial from the first call would show), each compared bit for bit
with kiv_decode_attention on the same inputs (the same kernels and split
layout) and with fp64 softmax attention to the attention bar.  A shape
whose partials exceed the static array is refused before any device work.
"""

from __future__ import annotations

import ctypes as C

import pytest
import torch

from kiv_amd import _native as nat
from kiv_amd import attention
from tests.test_gpu_retrieval import attention_check

pytestmark = pytest.mark.gpu


def _inputs(g, B, hq, hkv, D, P, T, dtype, device, masked):
    mk = lambda *s: torch.randn(*s, generator=g).to(dtype).to(device)
    q, ck, cv, hk, hv = mk(B, hq, 1, D), mk(B, hkv, P, D), mk(B, hkv, P, D), mk(B, hkv, T, D), mk(B, hkv, T, D)
    mask = (torch.rand(B, 1, 1, T, generator=g) > 0.3).to(device) if masked else None
    return q, ck, cv, hk, hv, mask


def _call(entry: str, q, ck, cv, hk, hv, mask, scaling, workspace: bool):
    args, out, _keep = attention._prepare(q, ck.shape[2], hk, hv, mask, scaling, workspace=workspace)
    attention._set_cold(args, ck, cv, q.dtype)
    rc = getattr(nat.lib(), entry)(C.byref(args), nat.stream_ptr(q.device))
    return rc, out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry(cuda, dtype):
    g = torch.Generator().manual_seed(71)
    shapes = [
        # B, Hq, Hkv, D, retrieved, hot, mask: a large call, then a smaller one
        (2, 28, 4, 128, 256, 2048, True),
        (1, 8, 2, 64, 37, 301, False),
    ]
    for B, hq, hkv, D, P, T, masked in shapes:
        print(f"noalloc {dtype} B={B} Hq={hq} Hkv={hkv} D={D} P={P} T={T} mask={masked}", flush=True)
        x = _inputs(g, B, hq, hkv, D, P, T, dtype, cuda, masked)
        scaling = D ** -0.5
        rc, got = _call("kiv_decode_attention_noalloc", *x, scaling, workspace=False)
        nat.check(rc, "kiv_decode_attention_noalloc")
        rc, ref = _call("kiv_decode_attention", *x, scaling, workspace=True)
        nat.check(rc, "kiv_decode_attention")
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        q, ck, cv, hk, hv, mask = x
        attention_check(q, ck, cv, hk, hv, scaling, mask, out=got)


def test_noalloc_refuses_partials_beyond_the_static_array(cuda):
    lib = nat.lib()
    B, hq, hkv, D, P, T = 4, 32, 8, 128, 256, 16384
    need = lib.kiv_attention_workspace_size(B, hq, hkv, D, 1, P, T)
    assert need > 8 << 20
    x = _inputs(torch.Generator().manual_seed(72), B, hq, hkv, D, P, T, torch.bfloat16, cuda, False)
    rc, _ = _call("kiv_decode_attention_noalloc", *x, D ** -0.5, workspace=False)
    assert rc == 4  # KIV_ERR_UNSUPPORTED
    assert b"static buffer" in lib.kiv_last_error()
