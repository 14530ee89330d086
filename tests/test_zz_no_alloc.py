"""GPU test of the allocation-free routing plan (cdx_route_plan_noalloc).

Through the C-ABI (ctypes), two calls in a row, the second on fewer tokens and
experts than the first: each call's five outputs must equal, bit for bit, those of
cdx_route_plan (caller workspace) on the same inputs, and the C oracle's.  The
second call runs on the scratch the first one left behind, so it also shows that
nothing in the scratch has to start at zero.  Output buffers are pre-filled with -1
so that an entry the kernels fail to write is caught.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _buffers(T, E):
    i32 = dict(dtype=torch.int32, device="cuda")
    return {"expert_id": torch.full((T,), -1, **i32), "perm": torch.full((T,), -1, **i32),
            "inv_perm": torch.full((T,), -1, **i32), "counts": torch.full((E,), -1, **i32),
            "offsets": torch.full((E + 1,), -1, **i32)}


def _args(b):
    return (b["expert_id"].data_ptr(), b["perm"].data_ptr(), b["inv_perm"].data_ptr(), b["counts"].data_ptr(),
            b["offsets"].data_ptr())


def test_noalloc_plan_matches_workspace_plan(cdx, oracle):
    from complexity_deep import _native as nat
    lib = nat.lib()
    assert lib.cdx_route_noalloc_scratch_bytes() == 256 * 64 * 4
    stream = torch.cuda.current_stream().cuda_stream
    for T, E, V, seed in [(300_000, 64, 32000, 1), (5000, 8, 3000, 2)]:
        print(f"route_plan_noalloc T={T} E={E} V={V}", flush=True)
        g = torch.Generator().manual_seed(seed)
        ids = torch.randint(-5, V + 5, (T,), generator=g).cuda()
        tmap = torch.randint(0, E, (V,), generator=g).cuda()
        ws_bytes = lib.cdx_route_workspace_bytes(T, E)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
        a, b = _buffers(T, E), _buffers(T, E)
        rc = lib.cdx_route_plan(ids.data_ptr(), T, tmap.data_ptr(), V, E, *_args(a), ws.data_ptr(), ws_bytes, stream)
        assert rc == 0, lib.cdx_last_error()
        rc = lib.cdx_route_plan_noalloc(ids.data_ptr(), T, tmap.data_ptr(), V, E, *_args(b), stream)
        assert rc == 0, lib.cdx_last_error()
        torch.cuda.synchronize()
        ref = oracle.route_plan(ids.cpu().numpy(), tmap.cpu().numpy(), E)
        for k in a:
            assert torch.equal(a[k], b[k]), k
            np.testing.assert_array_equal(b[k].cpu().numpy().astype(np.int64), ref[k].astype(np.int64), err_msg=k)


def test_noalloc_plan_argument_errors(cdx):
    from complexity_deep import _native as nat
    lib = nat.lib()
    CDX_EINVAL, CDX_EUNSUPPORTED = -1, -2
    assert lib.cdx_route_plan_noalloc(16, 10, 16, 5, 65, 16, 16, 16, 16, 16, None) == CDX_EUNSUPPORTED
    assert b"E=65" in lib.cdx_last_error()
    assert lib.cdx_route_plan_noalloc(None, 10, 16, 5, 4, 16, 16, 16, 16, 16, None) == CDX_EINVAL
    assert lib.cdx_route_plan_noalloc(16, -1, 16, 5, 4, 16, 16, 16, 16, 16, None) == CDX_EINVAL
