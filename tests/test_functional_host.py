"""Host-side argument handling of the NovaNN-compatible operators (no GPU:
every case here raises before any device work, as the reference raises
ValueError for the same inputs, novann/functional.py:302-313, :325-344)."""
import numpy as np
import pytest

from novann_amd import functional as F
from novann_amd.module import Parameters, _pair


def test_pair_rules():
    assert F._pair(3) == (3, 3)
    assert F._pair((3, 5)) == (3, 5)
    assert F._pair("valid") == (0, 0)
    with pytest.raises(ValueError, match="'same'"):
        F._pair("same")
    with pytest.raises(ValueError, match="Unsupported"):
        F._pair("full")
    assert _pair(2) == (2, 2)


def test_conv2d_bad_padding_mode_raises_value_error():
    x = np.ones((1, 1, 8, 8), np.float32)
    w = Parameters(np.ones((2, 1, 3, 3), np.float32))
    with pytest.raises(ValueError, match="padding_mode"):
        F.conv2d(x, w, 3, padding=1, padding_mode="mirror")


def test_conv2d_same_padding_raises_value_error():
    x = np.ones((1, 1, 8, 8), np.float32)
    w = Parameters(np.ones((2, 1, 3, 3), np.float32))
    with pytest.raises(ValueError):
        F.conv2d(x, w, 3, padding="same")


def test_extras_requests_are_validated_first():
    """extras=True (the reference's training caches) is accepted; bad
    arguments still raise the reference's ValueError before any device work."""
    x = np.ones((1, 1, 8, 8), np.float32)
    w = Parameters(np.ones((2, 1, 3, 3), np.float32))
    with pytest.raises(ValueError, match="padding_mode"):
        F.conv2d(x, w, 3, padding=1, padding_mode="mirror", extras=True)
    with pytest.raises(ValueError, match="padding_mode"):
        F.max_pool2d(x, 2, 2, padding_mode="mirror", extras=True)
    with pytest.raises(ValueError):
        F.im2col(x, 3, padding="same")


def test_fuse_validates_the_layer_sequence():
    """fuse() takes [Linear|Conv2d] [BatchNorm] [ReLU], in that order (host logic)."""
    from novann_amd import module as M
    conv = M.Conv2d.__new__(M.Conv2d)   # no weights needed to check the sequence
    lin = M.Linear.__new__(M.Linear)
    f = M.fuse(conv, M.BatchNorm2d(4), M.ReLU())
    assert f.bn is not None and f.relu
    assert M.fuse(lin, M.ReLU()).bn is None
    with pytest.raises(TypeError):
        M.fuse(conv, M.BatchNorm1d(4))
    with pytest.raises(ValueError):
        M.fuse(conv, M.ReLU(), M.BatchNorm2d(4))
    bn = M.BatchNorm2d(3)
    assert bn.gamma.data.shape == (1, 3, 1, 1) and bn.running_var.shape == (1, 3, 1, 1)
    assert M.BatchNorm1d(5).running_mean.shape == (1, 5)


def test_storage_size_checks():
    """The host layer refuses buffers too small for the element count before
    any launch (a kernel would read or write past their end)."""
    import torch

    from novann_amd import quant
    quant._require_holds(torch.empty(4, dtype=torch.float32), "f32", 4, "x")
    quant._require_holds(torch.empty(3, dtype=torch.uint8), "e2m1", 5, "x")   # ceil(5/2) bytes
    quant._require_holds(torch.empty(2, dtype=torch.float32), "e4m3", 8, "x")  # bytes count
    with pytest.raises(ValueError, match="need"):
        quant._require_holds(torch.empty(3, dtype=torch.float32), "f32", 4, "x")
    with pytest.raises(ValueError, match="need"):
        quant._require_holds(torch.empty(2, dtype=torch.uint8), "e2m1", 5, "x")
    with pytest.raises(ValueError, match="need"):
        quant._require_holds(torch.empty(7, dtype=torch.int16), "f16", 8, "x")
