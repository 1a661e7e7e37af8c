"""tgs_flags_compact_noalloc (the index-list entry point that allocates
nothing: its scratch is a static device array) against tgs_flags_compact, bit
for bit, on two calls in a row, the second with a smaller input."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _compact(fn, flags):
    import torch
    n = flags.numel()
    out = torch.full((max(n, 1),), -7, dtype=torch.int32, device="cuda")
    cnt = C.c_int64(-1)
    from tinygs_amd import _lib
    _lib.check(fn(C.c_void_p(flags.data_ptr()), n, C.c_void_p(out.data_ptr()), C.byref(cnt), None))
    torch.cuda.synchronize()
    return out.cpu().numpy(), cnt.value


@pytest.mark.parametrize("sizes", [(3_000_001, 70_001), (2048 * 4096, 1)])
def test_noalloc_compact_matches_allocating_one(hip, sizes):
    import torch
    from tinygs_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(sizes[1])
    for k, n in enumerate(sizes):
        print(f"[noalloc] call {k}: n={n}", flush=True)
        f = rng.integers(0, 3, n).astype(np.uint8) * (rng.random(n) < 0.3)
        flags = torch.from_numpy(f.astype(np.uint8)).cuda()
        a, ca = _compact(L.tgs_flags_compact, flags)
        b, cb = _compact(L.tgs_flags_compact_noalloc, flags)
        want = np.nonzero(f)[0].astype(np.int32)
        assert ca == cb == len(want)
        assert np.array_equal(a, b)
        assert np.array_equal(b[:cb], want)


def test_noalloc_compact_refuses_beyond_maximum(hip):
    from tinygs_amd import _lib
    L = _lib.load()
    cnt = C.c_int64(-1)
    rc = L.tgs_flags_compact_noalloc(C.c_void_p(16), (1 << 26) + 1, C.c_void_p(16), C.byref(cnt), None)
    assert rc == 1 and b"at most" in L.tgs_last_error()
