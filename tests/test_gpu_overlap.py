"""Adam's rows without gradient updated on a second stream while the backward
runs (TrainStep overlap_adam, tgs_rasterizer_backward_rows, the Adam row
selection and TGS_ADAM_SAME_STEP).

* the backward-rows mask known after the forward equals the sparse backward's
  row mask, byte for byte (fp32 and fp16 images, with and without
  densification statistics);
* a step in two parts (unmarked rows, then marked rows with the same step
  count) gives the same parameter bits as one masked step, over several steps
  (so the moments agree too), with the step count on the host or the device;
* the flag combinations that cannot work are refused."""
import ctypes as C

import numpy as np
import pytest

from helpers import tile_centred_scene
from tinygs_amd import scenes

pytestmark = pytest.mark.gpu


def _mask(ptr, n):
    import torch
    from tinygs_amd import _lib
    out = torch.empty(n, dtype=torch.uint8, device="cuda")
    _lib.copy_device(ptr, n, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("image_dtype", ["float32", "float16"])
@pytest.mark.parametrize("densif", [False, True])
def test_backward_rows_equal_the_sparse_row_mask(hip, image_dtype, densif):
    import torch
    from tinygs_amd.train import TrainStep
    scene = scenes.config2(seed=11, n=6000, width=246, height=182)
    ts = TrainStep(scene, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=True,
                   overlap_adam=False, image_dtype=image_dtype)
    if densif:
        ts.ctx.densification_info = torch.zeros((scene.n, 4), dtype=torch.float32, device="cuda")
    print(f"[overlap] rows mask {image_dtype} densif={densif}", flush=True)
    for _ in range(2):
        ts.zero()
        ts.forward()
        ts.losses_and_grad()
        early = _mask(ts.rasterizer.backward_rows(), scene.n)
        ts.backward()
        after = _mask(ts.rasterizer.grad_row_mask(), scene.n)
        assert np.array_equal(early, after), int((early != after).sum())
        assert 0 < int(after.sum()) < scene.n
        ts.optimize()


def _run(scene, steps, **kw):
    import torch
    from tinygs_amd.train import TrainStep
    s = torch.cuda.Stream()
    ts = TrainStep(scene, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=True, stream=s,
                   **kw)
    with torch.cuda.stream(s):
        for _ in range(steps):
            ts.step()
    s.synchronize()
    return ts


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


@pytest.mark.parametrize("no_sync", [False, True])
@pytest.mark.parametrize("image_dtype", ["float32", "float16"])
def test_two_part_step_equals_one_masked_step(hip, no_sync, image_dtype):
    scene = tile_centred_scene()
    print(f"[overlap] two-part step no_sync={no_sync} {image_dtype}", flush=True)
    seq = _run(scene, 4, overlap_adam=False, no_sync=no_sync, image_dtype=image_dtype)
    ovl = _run(scene, 4, overlap_adam=True, no_sync=no_sync, image_dtype=image_dtype)
    a, b = seq.params(), ovl.params()
    for k in a:
        bad = _bits(a[k]) != _bits(b[k])
        assert not bad.any(), (k, int(bad.sum()))
    assert seq.optimizer.global_steps() == ovl.optimizer.global_steps() == 4
    if no_sync:
        assert ovl.optimizer.device_steps(ovl.stream) == 4


def test_row_selection_flags_are_checked(hip):
    import torch
    from tinygs_amd import _lib
    from tinygs_amd.train import TrainStep
    scene = tile_centred_scene()
    ts = TrainStep(scene, sparse_grads=True, overlap_adam=False)
    L = _lib.load()
    h = ts.optimizer._h
    ts.optimizer._rebind()
    mask = torch.zeros(scene.n, dtype=torch.uint8, device="cuda")
    mp = C.c_void_p(mask.data_ptr())
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    # repeating a step before any step
    assert L.tgs_adam_step_ex(h, 1.0, mp, _lib.TGS_ADAM_ROWS_MARKED | _lib.TGS_ADAM_SAME_STEP, s) == \
        _lib.TGS_ERR_STATE
    # a row selection without a mask; both selections at once
    assert L.tgs_adam_step_ex(h, 1.0, None, _lib.TGS_ADAM_ROWS_UNMARKED, s) == _lib.TGS_ERR_INVALID
    assert L.tgs_adam_step_ex(h, 1.0, mp, _lib.TGS_ADAM_ROWS_UNMARKED | _lib.TGS_ADAM_ROWS_MARKED, s) == \
        _lib.TGS_ERR_INVALID
    assert ts.optimizer.global_steps() == 0
    # the second part must repeat the first part's mode
    assert L.tgs_adam_step_ex(h, 1.0, mp, _lib.TGS_ADAM_ROWS_UNMARKED, s) == _lib.TGS_OK
    assert L.tgs_adam_step_ex(h, 1.0, mp, _lib.TGS_ADAM_ROWS_MARKED | _lib.TGS_ADAM_SAME_STEP |
                              _lib.TGS_ADAM_DEVICE_STEP, s) == _lib.TGS_ERR_STATE
    assert L.tgs_adam_step_ex(h, 1.0, mp, _lib.TGS_ADAM_ROWS_MARKED | _lib.TGS_ADAM_SAME_STEP, s) == _lib.TGS_OK
    assert ts.optimizer.global_steps() == 1
    torch.cuda.synchronize()
    # backward rows before any forward
    r = ts.rasterizer
    out = C.c_void_p()
    assert L.tgs_rasterizer_backward_rows(r._h, C.byref(out), s) == _lib.TGS_ERR_STATE
