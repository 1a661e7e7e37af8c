"""CPU-side checks of the product library: it is built, it loads, it exports
every entry point include/tinygs_amd.h declares, and the Python host mirror
refuses misuse the way the reference does. No GPU compute is issued."""
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    src = open(os.path.join(ROOT, "include", "tinygs_amd.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tgs_[a-z0-9_]+)\s*\(", src)))


def test_header_declarations_match_binding():
    from tinygs_amd import _lib
    declared = _declared_functions()
    assert len(declared) >= 25
    assert set(declared) == set(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    from tinygs_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libtinygs_amd.so not built (run __graft_entry__.build())")
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.tgs_version() >= 1


def test_factories_reject_unknown_types():
    from tinygs_amd import _lib
    import ctypes as C
    lib = _lib.load()
    h = C.c_void_p()
    assert lib.tgs_rasterizer_create(b"default", C.byref(h)) != 0
    assert b"Unknown rasterizer type" in lib.tgs_last_error()
    assert lib.tgs_loss_create(b"huber", C.byref(h)) != 0
    assert b"Unknown loss type" in lib.tgs_last_error()


def test_python_factories_raise_like_reference():
    from tinygs_amd import rasterizer, loss, optim
    with pytest.raises(RuntimeError, match="Unknown rasterizer type"):
        rasterizer.create_rasterizer("gsplat")
    with pytest.raises(RuntimeError, match="Unknown loss type"):
        loss.create_loss("l2")
    with pytest.raises(RuntimeError, match="Unknown optimizer type"):
        optim.create_optimizer("lion", None, None)


def test_camera_layout_is_glm_column_major():
    from tinygs_amd.core import GPUBatchInput
    K = np.array([[100.0, 0, 30.0], [0, 110.0, 20.0], [0, 0, 1]])
    w2c = np.eye(4)
    w2c[:3, 3] = [1.0, 2.0, 3.0]
    c = GPUBatchInput(64, 48, 0.1, 50.0, K, w2c).to_c()
    assert (c.K[0], c.K[4], c.K[6], c.K[7]) == (100.0, 110.0, 30.0, 20.0)
    assert (c.w2c[12], c.w2c[13], c.w2c[14]) == (1.0, 2.0, 3.0)


def test_image_layout_roundtrip():
    from tinygs_amd.image import ImageShape, from_hwc, to_hwc
    for (w, h) in [(64, 64), (61, 45), (1, 1), (800, 8), (17, 33)]:
        s = ImageShape(w, h)
        img = np.random.default_rng(0).random((h, w, 3)).astype(np.float32)
        buf = from_hwc(img, s)
        assert buf.size == s.padded_size
        assert np.array_equal(to_hwc(buf, s), img)
