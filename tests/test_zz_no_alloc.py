"""iron_decode_attn_noalloc (the entry point for callers that cannot allocate) against
iron_decode_attn with a caller workspace: bit-identical outputs on two calls in a row, the second
with a smaller input, in both accumulation modes; the size limit is checked before any launch."""

import ctypes

import pytest
import torch

from iron_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH = 4 << 20


def _case(B, H, KV, L, ctx, seed):
    g = torch.Generator().manual_seed(seed)
    D = 128
    q = torch.randn(B * H * D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(B * KV * L * D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B * KV * L * D, generator=g).to(torch.bfloat16).to(DEV)
    c = torch.tensor(ctx, dtype=torch.int32).to(DEV)
    return q, k, v, c


def _run(lib, case, B, H, KV, L, acc, noalloc):
    q, k, v, c = case
    D = 128
    out = torch.full((B * H * D,), 3.0, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), KV * L * D, L * D, D, c.data_ptr(), 0,
            out.data_ptr(), B, H, KV, D, L, ctypes.c_float(D ** -0.5), acc)
    if noalloc:
        rc = lib.iron_decode_attn_noalloc(*args, s)
    else:
        n = lib.iron_decode_attn_workspace(B, H, KV, D, L)
        ws = torch.zeros(n, dtype=torch.uint8, device=DEV)
        rc = lib.iron_decode_attn(*args, ws.data_ptr(), n, s)
    assert rc == _lib.IRON_OK, lib.iron_last_error()
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("acc", [_lib.IRON_ACCUM_F64, _lib.IRON_ACCUM_F32])
def test_noalloc_matches_workspace_entry_point(lib, acc):
    # first a large call (several splits: B=2, 32 heads, context 8192), then a smaller one
    for B, H, KV, L, ctx in [(2, 32, 8, 8192, [8192, 5000]), (1, 16, 8, 1024, [700])]:
        print(f"[case] noalloc acc={acc} B={B} H={H} KV={KV} L={L} ctx={ctx}", flush=True)
        assert lib.iron_decode_attn_workspace(B, H, KV, 128, L) <= SCRATCH
        case = _case(B, H, KV, L, ctx, seed=B * 1000 + L)
        want = _run(lib, case, B, H, KV, L, acc, noalloc=False)
        got = _run(lib, case, B, H, KV, L, acc, noalloc=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (B, H, L)


def test_noalloc_rejects_partials_beyond_the_scratch(lib):
    B, H, KV, L = 255, 8, 2, 128   # 510 workgroups per split: two splits of 4.24 MB
    assert lib.iron_decode_attn_workspace(B, H, KV, 128, L) > SCRATCH
    print(f"[case] noalloc rejects B={B} H={H} KV={KV} L={L}", flush=True)
    # real buffers of the declared shape (~17 MB), so that even a launch could not stray
    q, k, v, _ = _case(B, H, KV, L, [L] * B, seed=3)
    out = torch.zeros(B * H * 128, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    rc = lib.iron_decode_attn_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), KV * L * 128,
                                      L * 128, 128, None, L, out.data_ptr(), B, H, KV, 128, L,
                                      ctypes.c_float(0.088), 0, s)
    assert rc == _lib.IRON_ERR_WORKSPACE
    assert b"scratch" in lib.iron_last_error()
    torch.cuda.synchronize()
    assert not bool(out.view(torch.int16).any()), "a rejected call wrote its output"
