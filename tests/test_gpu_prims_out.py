"""Caller-supplied output buffers on the GPU path: wrong dtype, count, device
or layout raises before the C ABI is called; the right ones are filled with
the same bits as the library-allocated outputs."""
import numpy as np
import pytest
import torch

from mlrs_amd import prims

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_knn_out_buffers():
    g = torch.Generator(device="cpu").manual_seed(3)
    xq = torch.randn((10, 8), generator=g).to(DEV)
    xt = torch.randn((500, 8), generator=g).to(DEV)
    with pytest.raises(TypeError):
        prims.knn_topk(xq, xt, 4, out=(torch.empty((10, 4), dtype=torch.float64, device=DEV),
                                       torch.empty((10, 4), dtype=torch.int32, device=DEV)))
    with pytest.raises(ValueError):
        prims.knn_topk(xq, xt, 4, out=(torch.empty((10, 4), device=DEV),
                                       torch.empty((10, 3), dtype=torch.int32, device=DEV)))
    with pytest.raises(ValueError):
        prims.knn_topk(xq, xt, 4, out=(torch.empty((10, 4)), torch.empty((10, 4), dtype=torch.int32)))
    with pytest.raises(TypeError):
        prims.knn_topk(xq, xt, 4, out=(torch.empty((10, 4), device=DEV),
                                       torch.empty((10, 4), dtype=torch.int64, device=DEV)))
    d0, i0 = prims.knn_topk(xq, xt, 4)
    d1 = torch.empty((10, 4), device=DEV)
    i1 = torch.empty((10, 4), dtype=torch.int32, device=DEV)
    prims.knn_topk(xq, xt, 4, out=(d1, i1))
    torch.cuda.synchronize()
    assert torch.equal(d0, d1) and torch.equal(i0, i1.to(torch.int64))


def test_assign_pairwise_norm_out_buffers():
    x = torch.randn((300, 5), dtype=torch.float64, device=DEV)
    c = torch.randn((7, 5), dtype=torch.float64, device=DEV)
    with pytest.raises(TypeError):
        prims.kmeans_assign(x, c, sqdist=torch.empty(300, dtype=torch.float32, device=DEV))
    with pytest.raises(ValueError):
        prims.kmeans_assign(x, c, labels=torch.empty(299, dtype=torch.int32, device=DEV))
    with pytest.raises(TypeError):
        prims.kmeans_assign(x, c.to(torch.float32))
    with pytest.raises(ValueError):
        prims.pairwise_distance(x, c, out=torch.empty((300, 6), dtype=torch.float64, device=DEV))
    with pytest.raises(ValueError):
        prims.row_sqnorms(x, out=torch.empty(300, dtype=torch.float64))
    out = torch.empty(300, dtype=torch.float64, device=DEV)
    prims.row_sqnorms(x, out=out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), prims.row_sqnorms(x).cpu().numpy())
