"""One MatRIS evaluation captured as a HIP graph and replayed (opt-in).

For repeated evaluation of graphs whose index arrays stay fixed -- one structure evaluated
many times, a batch of cells, a relaxation or MD run that keeps its neighbour list -- the
whole evaluation (process_graphs, the forward, autograd forces and stress, the magmom
head) is recorded once with torch.cuda.graph and replayed with one launch.  The host no
longer issues the ~900 kernel launches of an evaluation one by one, so the GPU does not
wait for it after the evaluation's status read.

What a replay reads: the current values of every graph's atom_frac_coord, lattice and
neighbor_image tensors (in-place updates are picked up), with the index arrays and CSR
groupings of capture time.  The graphs' index tensors must not change: replay() compares
their index signatures with the ones recorded at capture and raises if any differs
(capture again then).  Results: the same output tensors on every replay (the graph's own
memory), valid until the next replay; clone what must outlive it.

The status word keeps its role: each replay ends with one read of it (the only host sync),
a graph index outside its range raises, and in the f16x3 arithmetic an fp16 range overflow
warns and returns an eager bf16x6 evaluation instead, as MatRIS.forward does.  The MFMA
arithmetic of the replay is the one in effect at capture.

Nothing recorded contains a memset node: the library clears its counters and flags with
kernels, and the evaluation's own zero tensors are torch fill kernels.
"""
from __future__ import annotations

import warnings

import torch

from . import ops


class CapturedEvaluation:
    """A captured MatRIS evaluation of fixed graphs; replay() returns its outputs."""

    def __init__(self, model, graphs, task: str = "efsm", warmup: int = 2):
        if not torch.cuda.is_available():
            raise RuntimeError("CapturedEvaluation needs a ROCm device")
        self.model, self.graphs, self.task = model, list(graphs), task
        self.device = next(model.parameters()).device
        self.mode = ops.get_mma_precision()
        # eager evaluations first: the per-graph topology, the weight packs and the atom
        # embeddings are built and remembered outside the capture
        for _ in range(max(1, warmup)):
            model(self.graphs, task=task)
        self.signatures = [g.index_signature() for g in self.graphs]
        torch.cuda.synchronize(self.device)
        ops.status_take(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.outputs = model._evaluate(self.graphs, task)
        torch.cuda.synchronize(self.device)

    def replay(self) -> dict:
        """Run the captured evaluation; returns its output dict (the keys of MatRIS.forward)."""
        for g, sig in zip(self.graphs, self.signatures):
            if g.index_signature() != sig:
                raise RuntimeError("CapturedEvaluation: a graph's index arrays changed since the capture; "
                                   "capture again")
        self.graph.replay()
        bits = ops.status_take(self.device)
        if bits & ops.STATUS_CSR_KEY:
            raise RuntimeError("MatRIS: a graph index is outside its range (atom, bond or angle index)")
        if bits & ops.STATUS_F16_RANGE and self.mode == "f16x3":
            warnings.warn("MatRIS: an activation exceeded the fp16 range of the f16x3 GEMMs; "
                          "the evaluation was redone eagerly in bf16x6", RuntimeWarning, stacklevel=2)
            with ops.mma_precision("bf16x6"):
                pred = self.model._evaluate(self.graphs, self.task)
            ops.status_take(self.device)
            return pred
        return self.outputs
