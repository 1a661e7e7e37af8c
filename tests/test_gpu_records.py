"""The fp32 blend backward's 2D-gradient records and their fixed summation
order (blend_backward.hip, preprocess_backward.hip; the reference sums with
float atomics, kernels_backward.cuh:907-926, in whatever order its warps
finish).

* The tile sort carries each instance's rank among its primitive's instances
  (the emission's order, which is tile order): the GPU's ranks equal the
  ranks computed from the oracle's sorted instance list.
* The record of the instance of rank k of primitive p sits at slot
  first_slot[p] + k: the marked slots are exactly those of the instances the
  backward runs, a tile's instances up to its last contributor
  (kernels_backward.cuh:714 skips the buckets past it).
* The per-primitive sums (keep_2d) equal, bit for bit, the numpy restatement
  of the kernel's order applied to the GPU's own records
  (helpers.library_order_sums: rank order up to 16 records; above, the
  16-lane split by 8-slot bytes and an xor butterfly), so the order is
  pinned, and the oracle restates the same order (orc.blend_backward).
* Two backwards after one forward, and two forward + backward passes, give
  bit-identical gradients: nothing depends on the order in which the
  buckets finish.
"""
import numpy as np
import pytest

from tinygs_amd import scenes

from helpers import gpu_render, instance_ranks, library_order_sums, marked_slots

pytestmark = pytest.mark.gpu


def _cases():
    return {"config2_20k": scenes.config2(seed=11, n=20000, width=320, height=240),
            "config3_60k": scenes.config3(seed=31, n=60000, width=480, height=270)}


CASES = _cases()


def _backward(run, gimg, keep_2d=True):
    import torch
    from tinygs_amd.core import Image
    ctx = run["ctx"]
    grads = run["g"].gradient_like()
    ctx.gaussians_grad = grads
    ctx.grad_output.image = Image(ctx.fwd_output.image.shape, "float32",
                                  torch.from_numpy(np.ascontiguousarray(gimg, np.float32)).cuda())
    run["r"].backward(ctx, assign=True, keep_2d=keep_2d)
    torch.cuda.synchronize()
    return [t.cpu().numpy().copy() for t in grads.tensors()]


@pytest.mark.parametrize("case", list(CASES))
def test_record_slots_and_fixed_order_sums(hip, orc, case):
    s = CASES[case]
    print(f"[records] {case}: N={s.n} {s.camera.width}x{s.camera.height}", flush=True)
    run = gpu_render(s)
    pre, bins, fwd = orc.render(s, "f")
    dv = run["dv"]
    assert np.array_equal(dv["instance_prims"].view(np.uint32), bins["inst_prim"])
    gimg = scenes.grad_image(9, s.camera.shape)
    _backward(run, gimg)
    dr = run["r"].debug_records()
    I = bins["n_instances"]
    n = s.n
    # ranks: the instance's position among its primitive's instances in instance order
    assert np.array_equal(dr["ranks"].astype(np.int64), instance_ranks(bins["inst_prim"], n))
    fs = dr["first_slot"]
    assert np.array_equal(fs[pre["n_touched"] > 0], orc.first_slots(pre, bins)[pre["n_touched"] > 0])
    # the marked slots: a tile's instances up to its last contributor (its
    # buckets below the tile maximum, cut at the maximum)
    ranges = bins["ranges"].reshape(-1, 2).astype(np.int64)
    live = np.zeros(I, bool)
    for t, (a, b) in enumerate(ranges):
        if b > a:
            live[a:a + min(b - a, int(fwd["tile_max"][t]))] = True
    ranks = instance_ranks(bins["inst_prim"], n)
    slots = fs[bins["inst_prim"]].astype(np.int64) + ranks
    want = np.sort(slots[live])
    g2d = run["r"].debug_grad2d()
    masks = g2d["record_masks"]
    got = marked_slots(dr["bits"], masks, fs, I)
    assert np.array_equal(got, want), (got.size, want.size)
    # ranks below 32 are marked in the mask word only, the others by slot only
    bits_set = np.unpackbits(dr["bits"].view(np.uint8), bitorder="little")[:I].astype(bool)
    assert not bits_set[slots[live & (ranks < 32)]].any()
    assert np.array_equal(np.nonzero(bits_set)[0], np.sort(slots[live & (ranks >= 32)]))
    print(f"[records] {want.size} records of {I} instances at their rank slots "
          f"({int((live & (ranks >= 32)).sum())} of rank 32 or more)", flush=True)
    # the sums: bit-exact with the restated order on the GPU's own records
    ref = library_order_sums(dr["records"], dr["bits"], masks, fs, pre["n_touched"], I)
    gpu = np.concatenate([g2d["grad_mean2d"].reshape(n, 2), g2d["absgrad"].reshape(n, 2),
                          g2d["grad_conic"].reshape(n, 3), g2d["grad_color"].reshape(n, 3),
                          g2d["alpha_sum"].reshape(n, 1)], axis=1)
    bad = gpu.view(np.uint32) != ref[:, :11].view(np.uint32)
    heavy = np.bincount(bins["inst_prim"][live], minlength=n) > 16
    print(f"[records] {int(heavy.sum())} primitives above 16 records", flush=True)
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:5])


@pytest.mark.parametrize("case", list(CASES))
def test_gradients_repeat_bit_for_bit(hip, case):
    s = CASES[case]
    gimg = scenes.grad_image(9, s.camera.shape)
    print(f"[records] determinism {case}", flush=True)
    run = gpu_render(s, with_debug=False)
    a = _backward(run, gimg, keep_2d=False)
    b = _backward(run, gimg, keep_2d=False)          # a second backward after the same forward
    run2 = gpu_render(s, with_debug=False)
    c = _backward(run2, gimg, keep_2d=False)         # a new forward and backward
    for x, y, z in zip(a, b, c):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
        assert np.array_equal(x.view(np.uint32), z.view(np.uint32))
