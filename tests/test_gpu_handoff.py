"""The grid-wide hand-off probe behind the persistent kernel's design measurements: every mode
completes its phases with no wait giving up (the error word stays zero), launch after launch on
one workspace."""

import pytest
import torch

from iron_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode,n", [(_lib.IRON_HANDOFF_TAGGED, 256),
                                    (_lib.IRON_HANDOFF_TAGGED, 2048),
                                    (_lib.IRON_HANDOFF_COUNTER, 256),
                                    (_lib.IRON_HANDOFF_FLAGS, 1024),
                                    (_lib.IRON_HANDOFF_XCD_L2, 256),
                                    (_lib.IRON_HANDOFF_XCD_L2, 640),
                                    (_lib.IRON_HANDOFF_XCD_AGENT, 640)])
def test_handoff_probe_completes(lib, mode, n):
    print(f"[case] handoff probe mode={mode} n={n}", flush=True)
    nbytes = lib.iron_handoff_probe_workspace(n)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    base = 0
    for _ in range(3):
        if mode == _lib.IRON_HANDOFF_COUNTER:
            ws.zero_()
        _lib.check(lib.iron_handoff_probe(mode, n, 64, base, ws.data_ptr(), nbytes,
                                          _lib.stream_handle()))
        torch.cuda.synchronize()
        base += 65
        err = ws[nbytes - 4096 + 256: nbytes - 4096 + 264].view(torch.int32).cpu()
        assert int(err[0]) == 0 and int(err[1]) == 0, f"a wait gave up: {err.tolist()}"
