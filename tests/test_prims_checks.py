"""Caller-supplied output buffers are checked before the C ABI is called (it
counts elements, not bytes, and writes through raw pointers) -- CPU only: the
checks run on tensor metadata, nothing is launched."""
import pytest
import torch

from mlrs_amd import prims

CPU = torch.device("cpu")


def test_check_out_accepts_the_expected_buffer():
    prims._check_out(torch.empty((4, 3), dtype=torch.float32), "out", (torch.float32,), 12, CPU)
    prims._check_out(torch.empty(12, dtype=torch.int32), "idx", prims._IDX_DTYPES, 12, CPU)


@pytest.mark.parametrize("t,dtypes,numel,exc,words", [
    (torch.empty(12, dtype=torch.float64), (torch.float32,), 12, TypeError, "must be torch.float32"),
    (torch.empty(11, dtype=torch.float32), (torch.float32,), 12, ValueError, "12 elements"),
    (torch.empty((3, 8), dtype=torch.float32)[:, :4], (torch.float32,), 12, ValueError, "contiguous"),
    (torch.empty(12, dtype=torch.int64), prims._IDX_DTYPES, 12, TypeError, "must be torch.int32"),
    ([0.0] * 12, (torch.float32,), 12, TypeError, "must be a tensor"),
])
def test_check_out_rejects(t, dtypes, numel, exc, words):
    with pytest.raises(exc) as e:
        prims._check_out(t, "out", dtypes, numel, CPU)
    assert words in str(e.value)


def test_check_out_rejects_another_device():
    with pytest.raises(ValueError) as e:
        prims._check_out(torch.empty(12), "out", (torch.float32,), 12, torch.device("cuda:0"))
    assert "must be on cuda:0" in str(e.value)


def test_host_operands_are_rejected():
    x = torch.zeros((4, 3))
    with pytest.raises(ValueError) as e:
        prims.knn_topk(x, x, 2)
    assert "device tensors" in str(e.value)
