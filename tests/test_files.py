"""Graph files and model checkpoints (the on-disk formats of radiusgraph.py:115-160 and
model.py:256-317), CPU only: no kernel runs.

  * RadiusGraph.save / from_file round trip every field bit for bit;
  * a graph file written by the REFERENCE's own RadiusGraph.save (tests/golden/c1_graph_ref.pt,
    made by tests/golden/make_golden.py --only graphfile) loads with weights_only=True and
    holds the reference's C1 graph arrays (tests/golden/c1_cu4.npz);
  * a {"config", "state_dict"} checkpoint loads through MatRIS.load(path=...) /
    MatRIS.from_dict, and the loaded seed-0 weights are the reference's seed-0 weights
    (per-tensor sha256 of tests/golden/state_dict_seed0.json).
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from matris_amd.config import MATRIS_10M
from matris_amd.graph import RadiusGraph

from conftest import GOLDEN


def _c1_graph(z):
    t = lambda k, dt: torch.as_tensor(np.asarray(z[f"g_{k}"]), dtype=dt)
    return RadiusGraph(graph_id="c1", mp_id=None, composition="Cu4", atomic_number=t("z", torch.int32),
                       atom_frac_coord=t("frac", torch.float32), lattice=t("lattice", torch.float32),
                       neighbor_image=t("image", torch.float32), atom_graph=t("atom_graph", torch.int32),
                       atom_graph_cutoff=6.0, line_graph=t("line_graph", torch.int32), line_graph_cutoff=4.0,
                       directed2undirected=t("d2u", torch.int32), undirected2directed=t("u2d", torch.int32))


def test_graph_save_from_file_round_trip(golden, tmp_path):
    g = _c1_graph(golden("c1_cu4.npz"))
    path = g.save(save_dir=str(tmp_path))
    assert os.path.basename(path) == "c1.pt"  # radiusgraph.py:139-144: graph_id names the file
    h = RadiusGraph.from_file(path)
    for f in RadiusGraph._FIELDS:
        a, b = getattr(g, f), getattr(h, f)
        assert a.dtype == b.dtype and torch.equal(a, b), f
    assert (h.graph_id, h.composition, h.atom_graph_cutoff, h.line_graph_cutoff) == ("c1", "Cu4", 6.0, 4.0)


def test_reference_written_graph_file_loads(golden):
    """The file the reference's RadiusGraph.save wrote for C1 loads (weights_only) into a
    RadiusGraph whose arrays are the reference graph arrays of the C1 fixture."""
    z = golden("c1_cu4.npz")
    g = RadiusGraph.from_file(os.path.join(GOLDEN, "c1_graph_ref.pt"))
    assert isinstance(g, RadiusGraph) and g.graph_id == "c1_cu4"
    for f, k in (("atom_graph", "atom_graph"), ("line_graph", "line_graph"), ("directed2undirected", "d2u"),
                 ("undirected2directed", "u2d"), ("atomic_number", "z")):
        assert np.array_equal(getattr(g, f).numpy().astype(np.int64), np.asarray(z[f"g_{k}"]).astype(np.int64)), f
    assert g.atom_graph.dtype == torch.int32 and g.line_graph.dtype == torch.int32  # converter.py:93-106
    assert np.array_equal(g.neighbor_image.numpy(), np.asarray(z["g_image"], np.float32))
    assert np.array_equal(g.lattice.numpy(), np.asarray(z["g_lattice"], np.float32))


def test_checkpoint_load_gives_reference_seed0_weights(tmp_path):
    from matris_amd.model import MatRIS
    torch.manual_seed(0)
    m = MatRIS(**MATRIS_10M)
    path = tmp_path / "MatRIS_10M_test.pth.tar"
    torch.save({"config": dict(MATRIS_10M), "state_dict": m.state_dict()}, path)
    loaded = MatRIS.load(path=str(path), device="cpu")
    with open(os.path.join(GOLDEN, "state_dict_seed0.json")) as fh:
        ref = json.load(fh)["tensors"]
    sd = loaded.state_dict()
    assert set(sd) == set(ref)
    for k, v in sd.items():
        t = v.detach().contiguous()
        assert list(t.shape) == ref[k]["shape"], k
        assert hashlib.sha256(t.numpy().tobytes()).hexdigest() == ref[k]["sha256"], k
    again = MatRIS.from_dict(torch.load(path, weights_only=True))
    assert all(torch.equal(a, b) for a, b in zip(again.state_dict().values(), sd.values()))


def test_missing_checkpoint_raises(tmp_path):
    from matris_amd.model import MatRIS
    with pytest.raises(FileNotFoundError):
        MatRIS.load(path=str(tmp_path / "absent.pth.tar"), device="cpu")


def test_graph_converter_from_dict_takes_the_reference_keyword():
    from matris_amd.graph.converter import GraphConverter
    gc = GraphConverter.from_dict(dict={"atom_graph_cutoff": 5.0, "line_graph_cutoff": 3.0, "algorithm": "fast"})
    assert gc.atom_graph_cutoff == 5.0 and gc.line_graph_cutoff == 3.0
