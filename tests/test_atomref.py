"""AtomRef (reference_energy.py:14-201), CPU: the composition energy against closed forms,
the least-squares fit against known weights, the pre-fitted tables' keys and layout."""
import numpy as np
import pytest
import torch

from matris_amd.model.atomref import AtomRef
from matris_amd.model.atomref_tables import TABLES


class _G:
    def __init__(self, z):
        self.atomic_number = torch.as_tensor(z, dtype=torch.int32)


def test_composition_energy_closed_forms():
    ref = AtomRef("mptrj")
    w = torch.tensor(TABLES["mptrj"])
    cu = _G([29] * 4)
    cu2o = _G([29, 29, 8])
    e = ref([cu, cu2o])
    assert e.shape == (2,)
    assert torch.allclose(e[0], w[28])                          # one element: its own entry
    assert torch.allclose(e[1], (2 * w[28] + w[7]) / 3)          # intensive: the atom fractions
    ext = AtomRef(None, is_intensive=False)
    with torch.no_grad():
        ext.fc.weight.copy_(w.view(1, -1))
    assert torch.allclose(ext([cu2o])[0], 2 * w[28] + w[7])      # extensive: the counts


def test_fit_recovers_weights():
    rng = np.random.default_rng(0)
    w = rng.normal(size=94).astype(np.float32)
    graphs = [_G(rng.integers(1, 95, size=int(rng.integers(5, 40)))) for _ in range(400)]
    ref = AtomRef(None, is_intensive=False)
    comp = np.stack([np.bincount(g.atomic_number.numpy() - 1, minlength=94) for g in graphs]).astype(np.float64)
    ref.fit(graphs, comp @ w)
    assert ref.fitted
    np.testing.assert_allclose(ref.fc.weight.view(-1).numpy(), w, rtol=2e-3, atol=2e-3)


def test_tables_and_layout():
    for k in ("mptrj", "omat", "mpa"):
        assert len(TABLES[k]) == 94
    assert TABLES["demo"] is TABLES["mptrj"]
    ref = AtomRef("OMat")
    assert list(ref.state_dict()) == ["fc.weight"] and ref.fc.weight.shape == (1, 94)
    assert not ref.fc.weight.requires_grad and ref.is_intensive and ref.fitted
    with pytest.raises(NotImplementedError):
        AtomRef("unknown")


def test_model_carries_reference_energy_like_the_reference():
    """The module sits at `reference_energy.fc.weight` and is built before the other modules
    (it draws random numbers at construction, as the reference's does)."""
    from matris_amd.model import MatRIS
    torch.manual_seed(0)
    m1 = MatRIS(num_layers=1, reference_energy="mptrj")
    torch.manual_seed(0)
    m0 = MatRIS(num_layers=1)
    sd1, sd0 = m1.state_dict(), m0.state_dict()
    assert sd1["reference_energy.fc.weight"].shape == (1, 94)
    assert set(sd1) - set(sd0) == {"reference_energy.fc.weight"}
    # the Linear(94, 1) consumed 94 draws first, so the other weights differ from a model
    # without it while their shapes agree
    k = "atom_embedding.embedding.weight"
    assert k in sd0 and sd0[k].shape == sd1[k].shape and not torch.equal(sd0[k], sd1[k])


def test_reference_method_names():
    """The reference's AtomRef methods: initialize_from_MPtrj / _OMat / _MPA load the same
    tables as initialize_from, and fit takes structures (atomic_numbers, as pymatgen's
    Structure) as well as graphs, by the reference's keyword."""
    for meth, key in (("initialize_from_MPtrj", "mptrj"), ("initialize_from_OMat", "omat"),
                      ("initialize_from_MPA", "mpa")):
        a, b = AtomRef(None), AtomRef(None)
        getattr(a, meth)()
        b.initialize_from(key)
        assert torch.equal(a.fc.weight, b.fc.weight) and a.fitted

    class _S:  # a structure-like object: a plain sequence of atomic numbers
        def __init__(self, z):
            self.atomic_numbers = tuple(int(v) for v in z)

    rng = np.random.default_rng(1)
    w = rng.normal(size=94).astype(np.float32)
    zs = [rng.integers(1, 95, size=int(rng.integers(5, 40))) for _ in range(400)]
    comp = np.stack([np.bincount(z - 1, minlength=94) for z in zs]).astype(np.float64)
    ref = AtomRef(None, is_intensive=False)
    ref.fit(structures_or_graphs=[_S(z) for z in zs], energies=comp @ w)
    np.testing.assert_allclose(ref.fc.weight.view(-1).numpy(), w, rtol=2e-3, atol=2e-3)
