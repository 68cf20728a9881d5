"""The opt-in captured evaluation (MatRIS.capture, matris_amd/model/capture.py): every
replay, with eager evaluations and host syncs between replays, equals the eager
evaluation of the same inputs bit for bit and the reference's golden outputs to the
north-star tolerances; positions updated in place are picked up; changed index arrays
are refused."""
import numpy as np
import pytest
import torch

from matris_amd.config import MATRIS_10M

pytestmark = pytest.mark.gpu


def _model():
    from matris_amd.model import MatRIS
    torch.manual_seed(0)
    return MatRIS(**MATRIS_10M).to("cuda").eval()


def _np(out):
    return dict(e=out["e"].detach().cpu().numpy().copy(),
                f=torch.cat([f.detach() for f in out["f"]]).cpu().numpy().copy(),
                s=torch.stack([s.detach() for s in out["s"]]).cpu().numpy().copy(),
                m=torch.cat([m.detach() for m in out["m"]]).cpu().numpy().copy())


def _same(a, b):
    return all(np.array_equal(a[k], b[k]) for k in "efsm")


def _golden_close(out, z):
    assert np.all(np.abs(out["e"] - z["e"]) <= 1e-5 * np.abs(z["e"]))
    assert np.max(np.abs(out["f"] - z["f"])) <= 1e-4
    assert np.max(np.abs(out["s"] - z["s"])) <= 1e-4 * np.max(np.abs(z["s"]))
    assert np.max(np.abs(out["m"] - z["m"])) <= 1e-4 * np.max(np.abs(z["m"]))


def test_c3_replays_equal_eager_and_golden(golden):
    from matris_amd import workloads as W
    z = golden("c3_cu864.npz")
    model = _model()
    g = model.graph_converter(W.c3_cu864())
    cap = model.capture([g], task="efsm")
    eager = _np(model([g], task="efsm"))
    _golden_close(eager, z)
    for r in range(4):
        rep = _np(cap.replay())
        assert _same(rep, eager), f"replay {r}"
        _golden_close(rep, z)
        torch.cuda.synchronize()
        assert _same(_np(model([g], task="efsm")), eager)  # eager work between the replays


def test_replay_reads_updated_positions():
    """Positions moved in place (by less than the neighbour list's margin: the same index
    arrays stay valid) give the eager result for the moved positions."""
    from matris_amd import workloads as W
    model = _model()
    g = model.graph_converter(W.c3_cu864())
    cap = model.capture([g], task="efsm")
    before = _np(cap.replay())
    gen = torch.Generator(device="cuda").manual_seed(7)
    g.atom_frac_coord.add_(1e-5 * torch.randn(g.atom_frac_coord.shape, device="cuda", generator=gen))
    rep = _np(cap.replay())
    assert not np.array_equal(rep["f"], before["f"])
    assert _same(rep, _np(model([g], task="efsm")))


def test_c4_batch_replay(golden):
    """The 64-cell C4 batch: replays equal the eager batch bit for bit, and both the
    reference's golden per-cell outputs."""
    from matris_amd import workloads as W
    z = golden("c4_batch64.npz")
    model = _model()
    graphs = [model.graph_converter(c) for c in W.c4_batch64()]
    cap = model.capture(graphs, task="efsm")
    eager = _np(model(graphs, task="efsm"))
    for _ in range(3):
        rep = _np(cap.replay())
        assert _same(rep, eager)
        torch.cuda.synchronize()
    _golden_close(rep, z)


def test_changed_index_arrays_are_refused():
    from matris_amd import workloads as W
    model = _model()
    g = model.graph_converter(W.c1_cu4())
    cap = model.capture([g], task="ef")
    cap.replay()
    g.line_graph = g.line_graph.clone()
    with pytest.raises(RuntimeError, match="index arrays changed"):
        cap.replay()


@pytest.mark.parametrize("over", [dict(distance_expansion="Gaussian", three_body_expansion="fourier",
                                       is_conservation=False),
                                  dict(graph_conv_mlp="MLP", norm_type="layer", max_n=3, max_l=3),
                                  dict(node_feat_dim=64, edge_feat_dim=64, three_body_feat_dim=64,
                                       mlp_hidden_dims=(64, 64), activation_type="gelu")],
                         ids=["gauss_fourier_direct", "mlp_ln_sh33", "dim64_gelu"])
def test_generic_option_paths_replay(golden, over):
    """Non-default constructor options (torch layers on the device between the library's
    kernels) captured and replayed: every replay, with eager evaluations and syncs between
    the replays, equals the eager evaluation to fp32 rounding (the generic paths' torch
    scatters add in no fixed order), for one structure and for a batch."""
    from matris_amd.config import DEFAULT_CONFIG
    from matris_amd.model import MatRIS
    zc, zs = golden("c1_cu4.npz"), golden("cells_small.npz")
    torch.manual_seed(0)
    model = MatRIS(**dict(DEFAULT_CONFIG, num_layers=2, **over)).to("cuda").eval()
    import sys, os
    sys.path.insert(0, os.path.dirname(__file__))
    from test_gpu_model import _graph_from_arrays
    for graphs in ([_graph_from_arrays(zc, "g_")], [_graph_from_arrays(zs, f"g{i}_") for i in range(3)]):
        cap = model.capture(graphs, task="efsm")
        eager = _np(model(graphs, task="efsm"))
        for r in range(3):
            rep = _np(cap.replay())
            for k in "efsm":
                scale = max(np.max(np.abs(eager[k])), 1e-30)
                # forces: 1e-7 eV/A absolute as well (C1's vanish by symmetry, so both are
                # rounding noise of ~1e-9 that the unordered scatters place differently)
                floor = 1e-7 if k == "f" else 1e-9
                assert np.max(np.abs(rep[k] - eager[k])) <= 1e-6 * scale + floor, (r, k)
            torch.cuda.synchronize()
            model(graphs, task="efsm")
