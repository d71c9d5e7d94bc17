"""Host-side logic of the device tape that needs no GPU: broadcast shape
rules (tensor.rs:575-592), one_hot (losses.rs:169-175) and the op tables."""
import numpy as np
import pytest

from rgpu_amd import autograd as A
from rgpu_amd import gpu as G


@pytest.mark.parametrize("a,b", [((3, 4), (4,)), ((2, 1, 4), (1, 3, 1)), ((5,), (2, 1, 5)), ((), (3, 2)),
                                 ((1,), (1,)), ((7, 1), (1, 9)), ((2, 3, 4, 5), (3, 1, 5))])
def test_broadcast_shapes_follow_numpy(a, b):
    assert A.broadcast_shapes(a, b) == np.broadcast_shapes(a, b)


def test_broadcast_shapes_reject_mismatch():
    with pytest.raises(ValueError):
        A.broadcast_shapes((3, 4), (2, 4))


def test_one_hot():
    y = A.one_hot([2, 0, 1], 3)
    assert y.dtype == np.float32
    assert np.array_equal(y, np.eye(3, dtype=np.float32)[[2, 0, 1]])
    with pytest.raises(IndexError):
        A.one_hot([3], 3)


def test_op_tables_match_the_header():
    text = open(G.LIB_PATH.replace("rgpu_amd/librtensor_hip.so", "include/rtensor_hip.h")).read()
    for name, code in G.UNARY.items():
        assert f"RT_U_{name.upper()} = {code}," in text or f"RT_U_{name.upper()} = {code} " in text, name
    for name, code in G.BINARY.items():
        assert f"RT_B_{name.upper()} = {code}" in text, name
    assert f"RT_LOSS_MAE = {G.LOSS_MAE}," in text
    assert f"RT_LOSS_SOFTMAX_XENT = {G.LOSS_SOFTMAX_XENT}," in text
    assert f"RT_LOSS_BCE = {G.LOSS_BCE}," in text
    assert f"RT_LOSS_SOFTMAX_XENT_LOGITS = {G.LOSS_SOFTMAX_XENT_LOGITS}," in text
    assert f"RT_LOSS_SOFTMAX_XENT_LOGITS_MEAN = {G.LOSS_SOFTMAX_XENT_LOGITS_MEAN} " in text
