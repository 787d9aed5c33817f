"""Drop-in API surface of ``Cpab`` that runs without a GPU: constructor checks
and assertion messages (cpab/cpab.py:311-320), solver parameters
(cpab.py:112-129), params fields, and the GPU-only guard of the transformer
(transformer.py:40)."""
import numpy as np
import pytest
import torch

from cpab import Cpab
from cpab.pytorch.transformer import CPAB_transformer
from cpab.pytorch.interpolation import interpolate


@pytest.mark.parametrize("args,msg", [
    (("x",), "tess_size must be a list or tuple"),
    (([1, 2, 3, 4],), "Only 1D, 2D, and 3D"),
    (([2.0, 2],), "All elements must be integers"),
    (([0, 2],), "All elements must be positive"),
])
def test_constructor_asserts(args, msg):
    with pytest.raises(AssertionError, match=msg):
        Cpab(*args)


def test_constructor_flag_types():
    with pytest.raises(AssertionError, match="zero_boundary"):
        Cpab([2, 2], zero_boundary=1)
    with pytest.raises(AssertionError, match="volume_perservation"):
        Cpab([2, 2], volume_perservation=None)
    with pytest.raises(AssertionError, match="override"):
        Cpab([2, 2], override="no")


def test_params_fields():
    T = Cpab([20, 20])
    p = T.get_params()
    assert p.nc == [20, 20] and p.ndim == 2 and p.nC == 1600 and p.params_pr_cell == 6
    assert p.Ashape == [2, 3] and p.D == 9600 and p.d == 1522 == T.get_theta_dim()
    assert p.nstepsolver == 50 and p.adaptive_substeps is False
    assert p.zero_boundary and not p.valid_outside and p.inc == [0.05, 0.05]
    assert T.get_basis().shape == (9600, 1522)
    assert "Theta size" in repr(T)


def test_set_solver_params():
    T = Cpab([4])
    T.set_solver_params(nstepsolver=20, adaptive_substeps=True)
    assert T.params.nstepsolver == 20 and T.params.adaptive_substeps is True
    with pytest.raises(AssertionError, match="positive"):
        T.set_solver_params(0)
    with pytest.raises(AssertionError, match="integer"):
        T.set_solver_params(10.0)
    with pytest.raises(AssertionError, match="bool"):
        T.set_solver_params(10, 1)


def test_cpu_tensors_rejected():
    T = Cpab([3, 3])
    with pytest.raises(AssertionError, match="Only GPU tensors supported"):
        CPAB_transformer(torch.zeros(2, 10), torch.zeros(1, T.params.d), T.params)
    with pytest.raises(RuntimeError, match="only GPU"):
        interpolate(2, torch.zeros(1, 1, 4, 4), torch.zeros(1, 2, 16), [4, 4])


def test_transform_grid_batch_assert():
    T = Cpab([3, 3])
    with pytest.raises(AssertionError, match="first dimension must match theta"):
        T.transform_grid(torch.zeros(2, 2, 10), torch.zeros(3, T.params.d))


def test_chain_asserts():
    T = Cpab([3, 3])
    with pytest.raises(AssertionError, match="scale_by_dt must be bool"):
        T.transform_grid_chain(torch.zeros(2, 4), torch.zeros(2, T.params.d), scale_by_dt=1)
    with pytest.raises(AssertionError, match="theta_chain must have shape"):
        T.transform_grid_chain(torch.zeros(2, 4), torch.zeros(T.params.d))
    with pytest.raises(AssertionError, match="expected d="):
        T.transform_grid_chain(torch.zeros(2, 4), torch.zeros(2, 5))
    with pytest.raises(AssertionError, match="at least one transform"):
        T.transform_grid_chain(torch.zeros(2, 4), torch.zeros(0, T.params.d))


def test_interpolate_other_ndim_returns_none():
    assert interpolate(4, None, None, None) is None


def test_cell_centers():
    T = Cpab([2, 2])
    c = T.tesselation.get_cell_centers()
    assert c.shape == (16, 2)
    # cell 0: triangle (centre (0.25, 0.25), (0, 0), (0.5, 0))
    np.testing.assert_allclose(c[0], [0.25, 0.25 / 3], atol=1e-12)


def test_fused_paths_reject_cpu_tensors():
    from cpab.pytorch.transformer import CPAB_chain_transformer, CPAB_transform_data
    T = Cpab([3, 3])
    with pytest.raises(AssertionError, match="Only GPU tensors supported"):
        CPAB_chain_transformer(torch.zeros(2, 10), torch.zeros(2, 1, T.params.d), T.params)
    with pytest.raises(AssertionError, match="Only GPU tensors supported"):
        CPAB_transform_data(torch.zeros(1, 1, 4, 4), torch.zeros(1, T.params.d),
                            torch.zeros(8), [4, 4], T.params)


def test_transform_data_checks_before_device_work():
    # The fused transform_data validates shapes on the host and raises
    # RuntimeError (as the reference's TORCH_CHECKs do) before any launch.
    from cpab.pytorch import transformer as tr
    T = Cpab([3, 3])
    with pytest.raises(RuntimeError, match="theta must be"):
        tr._CPABImageFunction.forward(_Ctx(), torch.zeros(2, 1, 4, 4), torch.zeros(3, T.params.d),
                                      torch.zeros(8), [4, 4], T.params)
    with pytest.raises(RuntimeError, match="per-axis coordinates"):
        tr._CPABImageFunction.forward(_Ctx(), torch.zeros(2, 1, 4, 4), torch.zeros(2, T.params.d),
                                      torch.zeros(2, 16), [4, 4], T.params)
    with pytest.raises(RuntimeError, match="float32"):
        tr._CPABImageFunction.forward(_Ctx(), torch.zeros(2, 1, 4, 4, dtype=torch.float64),
                                      torch.zeros(2, T.params.d), torch.zeros(8), [4, 4],
                                      T.params)


class _Ctx:
    needs_input_grad = (False, False, False, False, False)

    def save_for_backward(self, *a):
        pass
