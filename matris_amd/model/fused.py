"""Line-graph layers of the interaction block as single autograd nodes with an explicit
backward.

The line graph carries the A three-body rows (A >> E >> N), so every elementwise pass
over [A, 128] tensors costs a full HBM round trip.  Here the residual updates, the
envelope weighting and every gradient accumulation live inside the kernels
(residual outputs of the gated-MLP / FFN epilogues, source-0 gradient accumulation in
the gated-MLP backward, a base term in the attention backward, the fused envelope
aggregation), so no [A, 128] tensor is touched by a separate elementwise kernel in
either direction.  Only input gradients are produced (forces and stress need no
parameter gradients).

Reference: matris/model/interaction_block.py:17-143 (Graph_Attention_Layer, line graph
branch) and :146-278 (Refinement, graph_type="line graph").
"""
from __future__ import annotations

import torch

from . import ops
from .ops import D

__all__ = ["line_attention", "line_refinement", "line_attention_fusable", "line_refinement_fusable",
           "checkpoint_needed", "shared_grad"]

# Approximate saved-activation bytes per interaction block when nothing is recomputed:
# per angle, line attention p_e, z_e [256] + a_s, a_t, e [128] and line refinement
# p_h, z_h [256] + h, edge-FFN pre-activation [128], plus the block's angle output
# [128]; per directed edge, the atom-graph layers' autograd tape (gated-MLP
# pre-activations, attention logits, gathers, FFN) -- about 16 [E_d, 128] tensors (fp32).
SAVED_BYTES_PER_ANGLE_BLOCK = 4 * (2 * 256 + 3 * 128 + 2 * 256 + 2 * 128 + 128)
SAVED_BYTES_PER_EDGE_BLOCK = 4 * 16 * 128


_DEVICE_BYTES: dict = {}


def _device_bytes(device) -> int:
    """The device's memory capacity (queried once per device)."""
    idx = torch.device(device).index if device is not None else None
    if idx is None:
        idx = torch.cuda.current_device()
    if idx not in _DEVICE_BYTES:
        _DEVICE_BYTES[idx] = torch.cuda.get_device_properties(idx).total_memory
    return _DEVICE_BYTES[idx]


def blocks_to_checkpoint(n_angles: int, n_edges: int, n_blocks: int, device=None,
                         total_bytes: int | None = None) -> int:
    """How many leading interaction blocks to checkpoint (keep their inputs, rerun their
    forward in the backward): none when the whole model's saved activations fit in 55% of
    the device's memory (total_bytes, default: the device's capacity), otherwise all but
    as many trailing blocks as fit there.  The trailing blocks' backward runs first and
    frees their activations before any checkpointed block is recomputed, so keeping k of
    them raises the peak over full checkpointing only when k exceeds one.  The reference
    checkpoints its two line-graph layers above 60,000 angles regardless of memory
    (interaction_block.py:15, :400-413)."""
    total = total_bytes if total_bytes is not None else _device_bytes(device)
    per_block = n_angles * SAVED_BYTES_PER_ANGLE_BLOCK + n_edges * SAVED_BYTES_PER_EDGE_BLOCK
    budget = 0.55 * total
    if n_blocks * per_block <= budget:
        return 0
    return n_blocks - min(n_blocks, int(budget // per_block))


def checkpoint_needed(n_angles: int, n_edges: int, n_blocks: int, device=None, total_bytes: int | None = None) -> bool:
    """Whether any interaction block is checkpointed (blocks_to_checkpoint > 0)."""
    return blocks_to_checkpoint(n_angles, n_edges, n_blocks, device, total_bytes) > 0


# ------------------------------------------------------------------------------------
# one gradient buffer for a tensor read by several fused layers
# ------------------------------------------------------------------------------------
class GradAccumulator:
    """The gradient of a tensor that several fused layers read (the smooth basis of every
    block's Refinement, a block's attended atom features), built in one buffer: the first
    layer's backward writes it, later ones add to it inside their kernels, so autograd
    issues no separate add per extra reader."""
    __slots__ = ("buf",)

    def __init__(self):
        self.buf = None


class _GradSink(torch.autograd.Function):
    """y = x, with y's fused readers leaving their x-gradients in a GradAccumulator; the
    backward returns that buffer plus whatever reached y through autograd itself."""

    @staticmethod
    def forward(ctx, x, acc):
        ctx.acc = acc
        ctx.set_materialize_grads(False)
        return x.view_as(x)

    @staticmethod
    def backward(ctx, g):
        buf, ctx.acc.buf = ctx.acc.buf, None
        if g is not None:
            buf = g if buf is None else buf + g
        return buf, None


def shared_grad(x: torch.Tensor) -> torch.Tensor:
    """x itself, marked so that the fused layers reading it accumulate their x-gradients in
    one buffer (the Refinements' basis and atom inputs).  Readers that are not fused
    layers return their gradients through autograd as usual; the two are added."""
    if not (torch.is_grad_enabled() and x.requires_grad):
        return x
    acc = GradAccumulator()
    y = _GradSink.apply(x, acc)
    y._matris_grad_acc = acc
    return y


def _acc_of(t):
    return getattr(t, "_matris_grad_acc", None)


def _acc_out(acc):
    """(out, accumulate) for a kernel writing this reader's gradient: the accumulator's
    buffer to add to, or a new output when it is empty or there is none."""
    if acc is None or acc.buf is None:
        return None, False
    return acc.buf, True


def _acc_keep(acc, g):
    """Leave g (the reader's gradient, already added to acc.buf when that existed) in the
    accumulator; returns what the reader hands autograd (None when acc took it)."""
    if acc is None:
        return g
    acc.buf = g
    return None


def _acc_add(acc, g):
    """g computed on its own: added to the accumulator (or kept as its first term)."""
    if acc is None:
        return g
    if acc.buf is None:
        acc.buf = g
    else:
        acc.buf.add_(g)
    return None


def _zeros_if_none(g, like):
    return ops._rows(like.shape[0], like.shape[1], like.device).zero_() if g is None else ops._f32c(g)


def _ffn_fusable(mlp) -> bool:
    L = mlp.layers
    return (len(L) == 4 and L[0].bias is None and L[3].bias is None and tuple(L[0].weight.shape) == (D, D)
            and tuple(L[3].weight.shape) == (D, D) and type(L[1]).__name__ == "FusedSiLU"
            and not getattr(mlp, "use_fp16", False)
            and all(l.p == 0.0 or not l.training for l in L if isinstance(l, torch.nn.Dropout)))


def _gmlp_fusable(m) -> bool:
    """A GatedMLP in the form the fused kernels implement (an MLP-and-norm update of
    graph_conv_mlp="MLP" is not one)."""
    f = getattr(m, "_fusable", None)
    return f is not None and f()


def _res_ok(w) -> bool:
    return tuple(w.shape) == (1, D)


def _env_wt(layer):
    """The learnable envelope's weight transposed, [K, 128] (kept per weight version)."""
    return layer._env.get(layer.learnable_envelope.weight).mats["wt0"]


def _runs(grp: ops.Grouping, blk: int):
    """(key, blk) for gmlp_bwd_raw's tile-run sums when grp's rows ascend by key (no
    permutation), else None (the block leaves as rows)."""
    return (grp.key, blk) if grp.perm is None else None


def _tile_rows(grp: ops.Grouping) -> int:
    return ops.gmlp_tile_rows() if grp.perm is None else 0


def line_attention_fusable(layer) -> bool:
    s, t = layer.source_weight_linear, layer.target_weight_linear
    return (_gmlp_fusable(layer.edge_nonlinear_update) and _gmlp_fusable(layer.node_nonlinear_update)
            and tuple(s.weight.shape) == (D, D) and s.bias is None and tuple(t.weight.shape) == (D, D)
            and t.bias is None and _res_ok(layer.node_res_weight) and _res_ok(layer.edge_res_weight))


# the envelope kernels (matris_env_linear, matris_env_agg_bwd_env_proj, matris_seg_sum_mul_proj)
# take at most this many basis functions per row
ENV_BASIS_MAX = 8


def _env_ok(layer) -> bool:
    env = layer.learnable_envelope
    return env.bias is None and env.in_features <= ENV_BASIS_MAX and env.out_features == D


def line_refinement_fusable(layer) -> bool:
    return (layer.graph_type == "line graph" and _gmlp_fusable(layer.edge_nonlinear_update) and _env_ok(layer)
            and _ffn_fusable(layer.node_FFN) and _ffn_fusable(layer.edge_FFN)
            and _res_ok(layer.node_res_weight) and _res_ok(layer.edge_res_weight))


def _attn_fwd(layer, bond, tb, lg, mode, save: bool):
    """Forward of the line attention.  Returns (bond', tb', saved tuple or None)."""
    tgt, src = lg["grp_tgt"], lg["grp_src"]
    A, E = tb.shape[0], bond.shape[0]
    r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
    pe = layer.edge_nonlinear_update._pack.get(layer.edge_nonlinear_update)
    pn = layer.node_nonlinear_update._pack.get(layer.node_nonlinear_update)
    pp = layer._proj.get(layer.source_weight_linear.weight, layer.target_weight_linear.weight)
    # the logit projections W_s tb, W_t tb ride the edge update's launch, which reads tb anyway
    e, p_e, z_e, tb_new, a_s, a_t = ops.gmlp_fwd_pair_raw(pe, [tb, bond, bond], [None, tgt.key, src.key], A, mode,
                                                          (tb, r_e), pp, save=save)
    y_t, y_s, lse_t, lse_s = ops.attn_fwd_raw(a_t, a_s, e, tgt, src, None)
    if not save:
        del a_s, a_t
    _, p_n, z_n, bond_new = ops.gmlp_fwd_raw(pn, [bond, y_t, y_s], [None, None, None], E, mode, res=(bond, r_n),
                                             save=save)
    saved = (p_e, z_e, a_s, a_t, e, y_t, y_s, lse_t, lse_s, p_n, z_n) if save else None
    return bond_new, tb_new, saved


class _LineAttention(torch.autograd.Function):
    """Graph_Attention_Layer on the line graph (bonds = nodes, angles = edges):
        e     = GatedMLP_e([tb, bond[tgt], bond[src]])                 [A]
        y_t, y_s = attention(W_t tb, W_s tb, e; tgt, src)              [E]
        n     = GatedMLP_n([bond, y_t, y_s])                           [E]
        bond' = n + r_n * bond,  tb' = e + r_e * tb
    With recompute, only (bond, tb) are kept and the forward runs again inside the
    backward (the reference's activation checkpointing of this layer for large A,
    interaction_block.py:15,400-413)."""

    @staticmethod
    def forward(ctx, bond, tb, layer, lg, recompute):
        ops._check_dev(bond, tb)
        bond, tb = ops._f32c(bond), ops._f32c(tb)
        mode = ops._MMA["mode"]
        bond_new, tb_new, saved = _attn_fwd(layer, bond, tb, lg, mode, save=not recompute)
        ctx.save_for_backward(bond, tb) if recompute else ctx.save_for_backward(*saved)
        ctx.mode, ctx.layer, ctx.lg, ctx.recompute = mode, layer, lg, recompute
        return bond_new, tb_new

    @staticmethod
    def backward(ctx, g_bond_new, g_tb_new):
        layer, lg, mode = ctx.layer, ctx.lg, ctx.mode
        if ctx.recompute:
            bond, tb = ctx.saved_tensors
            _, _, saved = _attn_fwd(layer, bond, tb, lg, mode, save=True)
        else:
            saved = ctx.saved_tensors
        p_e, z_e, a_s, a_t, e, y_t, y_s, lse_t, lse_s, p_n, z_n = saved
        pe = layer.edge_nonlinear_update._pack.get(layer.edge_nonlinear_update)
        pn = layer.node_nonlinear_update._pack.get(layer.node_nonlinear_update)
        pp = layer._proj.get(layer.source_weight_linear.weight, layer.target_weight_linear.weight)
        r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
        tgt, src = lg["grp_tgt"], lg["grp_src"]
        E = p_n.shape[0]
        g_bond_new = _zeros_if_none(g_bond_new, y_t)
        g_tb_new = _zeros_if_none(g_tb_new, e)
        # node update: g_bond = r_n g + dGatedMLP_n/dbond, g_y = [g_yt | g_ys]
        g_bond = ops._rows(E, D, e.device)
        g_y = ops.gmlp_bwd_raw(pn, g_bond_new, p_n, z_n, 3 * D, mode, g_x0=g_bond, acc0=False, res_w=r_n)
        del p_n, z_n
        # attention: g_e = g_tb_new (residual branch) + attention term.  Edge update: source
        # 0's (tb) gradient to g_tb, the bond gathers' to g_x (the target-bond block, rows
        # ascending by target, as tile-run partial sums).
        if mode != 6:
            # the attention's backward and the logit projections' in one launch: g_e, and
            # g_tb = g_as W_s + g_at W_t + r_e g_tb_new (the logit gradients stay on chip),
            # to which the GatedMLP backward adds tb's gradient
            g_e, g_tb = ops.attn_pair_bwd_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_y, tgt, src, g_tb_new, pp, r_e,
                                              mode)
            del a_t, a_s, e, saved
            g_x = ops.gmlp_bwd_raw(pe, g_e, p_e, z_e, 3 * D, mode, g_x0=g_tb, acc0=True, runs=_runs(tgt, 1))
            del g_e, p_e, z_e
        else:
            g_at, g_as, g_e = ops.attn_bwd_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_y, g_y[:, D:], tgt, src, None,
                                               ldgy=2 * D, g_e_base=g_tb_new)
            del a_t, a_s, e, saved
            g_tb = ops._rows(p_e.shape[0], D, p_e.device)
            g_x = ops.gmlp_bwd_raw(pe, g_e, p_e, z_e, 3 * D, mode, g_x0=g_tb, acc0=False, runs=_runs(tgt, 1))
            del g_e, p_e, z_e
            # projections + residual, added to g_tb by the pair kernel (which stores nothing
            # before its read-modify-write of g_tb)
            ops.pair_bwd_raw(pp, g_as, g_at, mode, res=g_tb_new, res_w=r_e, out=g_tb, accumulate=True)
            del g_as, g_at
        ops.seg_sum_raw(g_x, tgt, ldx=2 * D, col_off=0, out=g_bond, accumulate=True,
                        second=(g_x, src, 1.0, 2 * D, D), tile_rows=_tile_rows(tgt))
        return g_bond, g_tb, None, None, None


def _refine_fwd(layer, tb, atom, bond, env, lg, mode, save: bool):
    """Forward of the line refinement.  Returns (bond', tb', saved tuple or None)."""
    tgt, src, grp_atom = lg["grp_tgt"], lg["grp_src"], lg["grp_atom"]
    A = tb.shape[0]
    r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
    ph = layer.edge_nonlinear_update._pack.get(layer.edge_nonlinear_update)
    L, M = layer.node_FFN.layers, layer.edge_FFN.layers
    pn = layer._node_ffn.get(L[0].weight, L[3].weight)
    pm = layer._edge_ffn.get(M[0].weight, M[3].weight)
    # h = GatedMLP(...) and tb' = edge_FFN(h) + r_e tb in one launch
    h, p_h, z_h, tb_new, p_de = ops.gmlp_fwd_ffn_raw(ph, [tb, atom, bond, bond],
                                                     [None, grp_atom.key, tgt.key, src.key], A, mode, pm, tb, r_e,
                                                     save=save)
    agg, S = ops.env_agg_fwd_raw(h, env, tgt, src)
    bond_new, p_dn = ops.ffn_fwd_raw(pn, agg, mode, res=(bond, r_n), save=save)
    saved = (h, p_h, z_h, S, p_dn, p_de) if save else None
    return bond_new, tb_new, saved


class _LineRefinement(torch.autograd.Function):
    """Refinement on the line graph:
        h     = GatedMLP([tb, atom[atom_list], bond[tgt], bond[src]])   [A]
        agg   = sum_tgt h * env[src] * env[tgt]                           [E]
        bond' = node_FFN(agg) + r_n * bond,  tb' = edge_FFN(h) + r_e * tb
    With recompute, only the inputs are kept and the forward reruns in the backward."""

    @staticmethod
    def forward(ctx, tb, atom, bond, basis, layer, lg, recompute):
        ops._check_dev(tb, atom, bond, basis)
        ctx.acc_atom, ctx.acc_basis = _acc_of(atom), _acc_of(basis)
        tb, atom, bond, basis = (ops._f32c(t) for t in (tb, atom, bond, basis))
        mode = ops._MMA["mode"]
        env = ops.env_linear_raw(basis, _env_wt(layer))
        bond_new, tb_new, saved = _refine_fwd(layer, tb, atom, bond, env, lg, mode, save=not recompute)
        if recompute:
            ctx.save_for_backward(tb, atom, bond, env)
        else:
            ctx.save_for_backward(env, *saved)
        ctx.mode, ctx.layer, ctx.lg, ctx.recompute, ctx.n_atom = mode, layer, lg, recompute, atom.shape[0]
        # an unused output (the last block's three-body features) arrives as None, not as a
        # materialised [A, 128] zero tensor
        ctx.set_materialize_grads(False)
        return bond_new, tb_new

    @staticmethod
    def backward(ctx, g_bond_new, g_tb_new):
        layer, lg, mode = ctx.layer, ctx.lg, ctx.mode
        if ctx.recompute:
            tb, atom, bond, env = ctx.saved_tensors
            _, _, saved = _refine_fwd(layer, tb, atom, bond, env, lg, mode, save=True)
            del tb, atom, bond
        else:
            env, *saved = ctx.saved_tensors
        h, p_h, z_h, S, p_dn, p_de = saved
        del saved
        ph = layer.edge_nonlinear_update._pack.get(layer.edge_nonlinear_update)
        L, M = layer.node_FFN.layers, layer.edge_FFN.layers
        pn = layer._node_ffn.get(L[0].weight, L[3].weight)
        pm = layer._edge_ffn.get(M[0].weight, M[3].weight)
        r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
        tgt, src = lg["grp_tgt"], lg["grp_src"]
        E, A = env.shape[0], h.shape[0]
        g_bond_new = _zeros_if_none(g_bond_new, env)
        g_bond = ops._rows(E, D, h.device)
        g_agg = ops.ffn_bwd_raw(pn, g_bond_new, p_dn, mode, g_res=g_bond, res_w=r_n)
        # the envelope's gradient leaves projected onto its basis (the learnable envelope's
        # input gradient), so the [E, 128] g_env is never stored
        g_basis, g_agg_env = ops.env_agg_bwd_env_raw(h, env, g_agg, S, tgt, src, proj_wt=_env_wt(layer),
                                                     g_basis=_acc_out(ctx.acc_basis)[0])
        g_basis = _acc_keep(ctx.acc_basis, g_basis)
        del h
        # g_h = edge_FFN's input gradient + the aggregate's term; g_tb = source 0's
        # GatedMLP gradient + r_e g_tb_new.  In the two-plane modes g_h never leaves the
        # GatedMLP backward (its head computes it per tile).
        g_tb = ops._rows(A, D, env.device)
        if g_tb_new is None:
            # tb' unused: no edge_FFN or residual term, g_h is the aggregate's term alone
            g_h = ops.gather_mul_raw(g_agg_env, tgt.key, env, src.key, out=ops._rows(A, D, env.device))
            g_x = ops.gmlp_bwd_raw(ph, g_h, p_h, z_h, 4 * D, mode, g_x0=g_tb, acc0=False, runs=_runs(tgt, 2))
            del g_h
        elif mode != 6:
            g_x = ops.gmlp_bwd_ffn_raw(ph, p_h, z_h, 4 * D, mode, pm, g_tb_new, p_de, env_term=(g_agg_env, env, tgt, src),
                                       g_x0=g_tb, res_w=r_e, runs=_runs(tgt, 2))
        else:
            g_h = ops.ffn_bwd_raw(pm, g_tb_new, p_de, mode, env_term=(g_agg_env, env, tgt, src))
            g_x = ops.gmlp_bwd_raw(ph, g_h, p_h, z_h, 4 * D, mode, g_x0=g_tb, acc0=False, res_w=r_e,
                                   res_src=g_tb_new, runs=_runs(tgt, 2))
            del g_h
        del p_de, g_agg_env, p_h, z_h
        out, acc = _acc_out(ctx.acc_atom)
        g_atom = _acc_keep(ctx.acc_atom, ops.seg_sum_raw(g_x, lg["grp_atom"], ldx=3 * D, col_off=0, out=out,
                                                         accumulate=acc))
        ops.seg_sum_raw(g_x, tgt, ldx=3 * D, col_off=D, out=g_bond, accumulate=True,
                        second=(g_x, src, 1.0, 3 * D, 2 * D), tile_rows=_tile_rows(tgt))
        return g_tb, g_atom, g_bond, g_basis, None, None, None


def line_attention(layer, bond, tb, lg, recompute: bool = False):
    """(bond', tb') of Graph_Attention_Layer.forward on the line graph."""
    return _LineAttention.apply(bond, tb, layer, lg, recompute)


def line_refinement(layer, tb, atom, bond, basis, lg, recompute: bool = False):
    """(bond', tb') of Refinement.forward on the line graph; basis = the smooth weights the
    learnable envelope maps to env (formed inside, matris_env_linear)."""
    return _LineRefinement.apply(tb, atom, bond, basis, layer, lg, recompute)


# ------------------------------------------------------------------------------------
# atom-graph layers (directed edges E_d, undirected bonds E_u via d2u, atoms N)
# ------------------------------------------------------------------------------------
def atom_attention_fusable(layer) -> bool:
    return line_attention_fusable(layer)


def atom_refinement_fusable(layer) -> bool:
    return (layer.graph_type == "atom graph" and _gmlp_fusable(layer.edge_nonlinear_update) and _env_ok(layer)
            and _ffn_fusable(layer.node_FFN) and _ffn_fusable(layer.edge_FFN)
            and _res_ok(layer.node_res_weight) and _res_ok(layer.edge_res_weight))


def _atom_packs(layer):
    pe = layer.edge_nonlinear_update._pack.get(layer.edge_nonlinear_update)
    pn = layer.node_nonlinear_update._pack.get(layer.node_nonlinear_update)
    pp = layer._proj.get(layer.source_weight_linear.weight, layer.target_weight_linear.weight)
    return pe, pn, pp


class _AtomAttention(torch.autograd.Function):
    """Graph_Attention_Layer on the atom graph (interaction_block.py:87-143 with
    is_atom_graph, called :416-422):
        e      = GatedMLP_e([bond[d2u], atom[tgt], atom[src]])            [E_d]
        y_t, y_s = attention(W_t bond[d2u], W_s bond[d2u], e; tgt, src)  [N]
        n      = GatedMLP_n([atom, y_t, y_s])                            [N]
        atom'  = n + r_n * atom,  bond' = mean_{d2u}(e) + r_e * bond     [E_u]
    The attention logits are computed once per undirected bond and read through d2u."""

    @staticmethod
    def forward(ctx, atom, bond, layer, ag, d2u):
        ops._check_dev(atom, bond)
        atom, bond = ops._f32c(atom), ops._f32c(bond)
        mode = ops._MMA["mode"]
        tgt, src = ag["grp_tgt"], ag["grp_src"]
        Ed, N = d2u.key.numel(), atom.shape[0]
        r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
        pe, pn, pp = _atom_packs(layer)
        e, p_e, z_e, _ = ops.gmlp_fwd_raw(pe, [bond, atom, atom], [d2u.key, tgt.key, src.key], Ed, mode)
        a_s, a_t = ops.pair_fwd_raw(pp, bond, mode)
        y_t, y_s, lse_t, lse_s = ops.attn_fwd_raw(a_t, a_s, e, tgt, src, d2u)
        _, p_n, z_n, atom_new = ops.gmlp_fwd_raw(pn, [atom, y_t, y_s], [None, None, None], N, mode, res=(atom, r_n))
        bond_new = ops.seg_sum_raw(e, d2u, 0.5, base=(bond, r_e))  # mean of the two directed copies + r_e bond
        ctx.save_for_backward(p_e, z_e, a_s, a_t, e, y_t, y_s, lse_t, lse_s, p_n, z_n)
        ctx.mode, ctx.layer, ctx.ag, ctx.d2u = mode, layer, ag, d2u
        return atom_new, bond_new

    @staticmethod
    def backward(ctx, g_atom_new, g_bond_new):
        layer, ag, d2u, mode = ctx.layer, ctx.ag, ctx.d2u, ctx.mode
        p_e, z_e, a_s, a_t, e, y_t, y_s, lse_t, lse_s, p_n, z_n = ctx.saved_tensors
        tgt, src = ag["grp_tgt"], ag["grp_src"]
        pe, pn, pp = _atom_packs(layer)
        r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
        N = p_n.shape[0]
        g_atom_new = _zeros_if_none(g_atom_new, y_t)
        g_bond_new = _zeros_if_none(g_bond_new, a_s)
        # node update: g_atom = r_n g + d GatedMLP_n / d atom; g_y = [g_yt | g_ys]
        g_atom = ops._rows(N, D, e.device)
        g_y = ops.gmlp_bwd_raw(pn, g_atom_new, p_n, z_n, 3 * D, mode, g_x0=g_atom, acc0=False, res_w=r_n)
        del p_n, z_n
        # by bond: g_e = half of the bond gradient of each directed copy + the attention
        # term; the logits were read through d2u, so their gradients are the bond's sums
        g_at, g_as, g_e = ops.attn_bwd_bond_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_y, g_y[:, D:], tgt, src, d2u,
                                                ldgy=2 * D, g_base=g_bond_new, base_scale=0.5)
        del g_y, a_t, a_s, e
        # the projections + residual
        g_bond = ops.pair_bwd_raw(pp, g_as, g_at, mode, res=g_bond_new, res_w=r_e)
        del g_at, g_as
        # edge update: sources bond[d2u], atom[tgt], atom[src]
        # the centre-atom block (rows ascend by centre) leaves as tile-run partial sums
        g_x = ops.gmlp_bwd_raw(pe, g_e, p_e, z_e, 3 * D, mode, runs=_runs(tgt, 1))
        del g_e, p_e, z_e
        ops.seg_sum_raw(g_x, d2u, ldx=3 * D, col_off=0, out=g_bond, accumulate=True)
        ops.seg_sum_raw(g_x, tgt, ldx=3 * D, col_off=D, out=g_atom, accumulate=True,
                        second=(g_x, src, 1.0, 3 * D, 2 * D), tile_rows=_tile_rows(tgt))
        return g_atom, g_bond, None, None, None


class _AtomRefinement(torch.autograd.Function):
    """Refinement on the atom graph (interaction_block.py:218-278 with is_atom_graph,
    called :437-446):
        w     = env[d2u]                                                  [E_d]
        h     = GatedMLP([bond[d2u], atom[tgt], atom[src]])               [E_d]
        atom' = node_FFN(sum_tgt h * w) + r_n * atom
        bond' = mean_{d2u} edge_FFN(h or h * w) + r_e * bond
    env = learnable_envelope(basis) [E_u], formed here (matris_env_linear); the backward
    returns the basis gradient."""

    @staticmethod
    def forward(ctx, atom, bond, basis, layer, ag, d2u):
        ops._check_dev(atom, bond, basis)
        ctx.acc_atom, ctx.acc_basis = _acc_of(atom), _acc_of(basis)
        atom, bond = ops._f32c(atom), ops._f32c(bond)
        env = ops.env_linear_raw(basis, _env_wt(layer))
        mode = ops._MMA["mode"]
        tgt, src = ag["grp_tgt"], ag["grp_src"]
        Ed = d2u.key.numel()
        r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
        ph = layer.edge_nonlinear_update._pack.get(layer.edge_nonlinear_update)
        L, Mm = layer.node_FFN.layers, layer.edge_FFN.layers
        pn = layer._node_ffn.get(L[0].weight, L[3].weight)
        pm = layer._edge_ffn.get(Mm[0].weight, Mm[3].weight)
        smoothed = bool(layer.use_smoothed_for_delta_edge)
        if smoothed:  # h * w also feeds the edge FFN: materialised
            h, p_h, z_h, _ = ops.gmlp_fwd_raw(ph, [bond, atom, atom], [d2u.key, tgt.key, src.key], Ed, mode)
            w = ops.gather_raw(env, d2u.key)
            hw = h * w
            agg = ops.seg_sum_raw(hw, tgt)
            de, p_de = ops.ffn_fwd_raw(pm, hw, mode)
        else:  # de = edge_FFN(h) in the GatedMLP's launch; sum_tgt h * env[d2u] in one pass
            h, p_h, z_h, de, p_de = ops.gmlp_fwd_ffn_raw(ph, [bond, atom, atom], [d2u.key, tgt.key, src.key], Ed,
                                                         mode, pm)
            w, hw = env, None
            agg = ops.seg_sum_mul_raw(h, tgt, env, d2u.key)
        atom_new, p_dn = ops.ffn_fwd_raw(pn, agg, mode, res=(atom, r_n))
        del hw, agg
        bond_new = ops.seg_sum_raw(de, d2u, 0.5, base=(bond, r_e))
        ctx.save_for_backward(w, h, p_h, z_h, p_dn, p_de)  # w = env[d2u] if smoothed, else env
        ctx.mode, ctx.layer, ctx.ag, ctx.d2u, ctx.smoothed = mode, layer, ag, d2u, smoothed
        ctx.set_materialize_grads(False)  # the last block's bond' is unused: its gradient is None
        return atom_new, bond_new

    @staticmethod
    def backward(ctx, g_atom_new, g_bond_new):
        layer, ag, d2u, mode = ctx.layer, ctx.ag, ctx.d2u, ctx.mode
        w, h, p_h, z_h, p_dn, p_de = ctx.saved_tensors
        tgt, src = ag["grp_tgt"], ag["grp_src"]
        ph = layer.edge_nonlinear_update._pack.get(layer.edge_nonlinear_update)
        L, Mm = layer.node_FFN.layers, layer.edge_FFN.layers
        pn = layer._node_ffn.get(L[0].weight, L[3].weight)
        pm = layer._edge_ffn.get(Mm[0].weight, Mm[3].weight)
        r_n, r_e = ops._vec(layer.node_res_weight), ops._vec(layer.edge_res_weight)
        N = p_dn.shape[0]
        g_atom_new = _zeros_if_none(g_atom_new, p_dn)
        g_atom = ops._rows(N, D, h.device)
        g_agg = ops.ffn_bwd_raw(pn, g_atom_new, p_dn, mode, g_res=g_atom, res_w=r_n)
        del p_dn
        if not ctx.smoothed and mode != 6:
            # g_h = edge_FFN's input gradient (from half the bond gradient of each directed
            # copy) + g_agg[tgt] * env[d2u], computed per tile inside the GatedMLP backward;
            # g_env = sum_{d2u} h * g_agg[tgt] leaves projected onto the envelope's basis
            g_basis = ops.seg_sum_mul_proj_raw(h, d2u, g_agg, tgt.key, _env_wt(layer),
                                               out=_acc_out(ctx.acc_basis)[0])
            g_basis = _acc_keep(ctx.acc_basis, g_basis)
            del h
            if g_bond_new is None:
                # bond' unused: no edge_FFN or residual term, g_h is the aggregate's term alone
                g_h = ops.gather_mul_raw(g_agg, tgt.key, w, d2u.key, out=ops._rows(d2u.key.numel(), D, w.device))
                g_x = ops.gmlp_bwd_raw(ph, g_h, p_h, z_h, 3 * D, mode, runs=_runs(tgt, 1))
                del g_h, p_h, z_h, p_de, w
                g_bond = ops.seg_sum_raw(g_x, d2u, ldx=3 * D, col_off=0)
            else:
                g_x = ops.gmlp_bwd_ffn_raw(ph, p_h, z_h, 3 * D, mode, pm, g_bond_new, p_de,
                                           env_term=(g_agg, w, tgt, d2u), runs=_runs(tgt, 1), ffn_g_idx=d2u.key,
                                           ffn_g_scale=0.5)
                del p_h, z_h, p_de, w
                g_bond = ops.seg_sum_raw(g_x, d2u, ldx=3 * D, col_off=0, base=(g_bond_new, r_e))
            ops.seg_sum_raw(g_x, tgt, ldx=3 * D, col_off=D, out=g_atom, accumulate=True,
                            second=(g_x, src, 1.0, 3 * D, 2 * D), tile_rows=_tile_rows(tgt))
            return _acc_add(ctx.acc_atom, g_atom), g_bond, g_basis, None, None, None
        g_bond_new = _zeros_if_none(g_bond_new, ops._rows(d2u.n_seg, D, h.device))
        g_te = ops.ffn_bwd_raw(pm, ops.gather_raw(g_bond_new, d2u.key, 0.5), p_de, mode)
        del p_de
        if ctx.smoothed:
            g_hw = ops.gather_raw(g_agg, tgt.key)
            g_hw += g_te
            g_h = g_hw * w
            g_env = ops.seg_sum_raw(g_hw * h, d2u)
            del g_hw
        else:  # g_h = g_te + g_agg[tgt] * env[d2u];  g_env = sum_d2u h * g_agg[tgt]
            g_h = ops.gather_mul_raw(g_agg, tgt.key, w, d2u.key, out=g_te, accumulate=True)
            g_env = ops.seg_sum_mul_raw(h, d2u, g_agg, tgt.key)
        del g_te, h, w
        g_x = ops.gmlp_bwd_raw(ph, g_h, p_h, z_h, 3 * D, mode, runs=_runs(tgt, 1))
        del g_h, p_h, z_h
        g_bond = ops.seg_sum_raw(g_x, d2u, ldx=3 * D, col_off=0, base=(g_bond_new, r_e))
        ops.seg_sum_raw(g_x, tgt, ldx=3 * D, col_off=D, out=g_atom, accumulate=True,
                        second=(g_x, src, 1.0, 3 * D, 2 * D), tile_rows=_tile_rows(tgt))
        return (_acc_add(ctx.acc_atom, g_atom), g_bond, _acc_add(ctx.acc_basis, g_env @ _env_wt(layer).t()), None,
                None, None)


def atom_attention(layer, atom, bond, ag, d2u):
    """(atom', bond') of Graph_Attention_Layer.forward on the atom graph."""
    return _AtomAttention.apply(atom, bond, layer, ag, d2u)


def atom_refinement(layer, atom, bond, basis, ag, d2u):
    """(atom', bond') of Refinement.forward on the atom graph; basis = the smooth weights the
    learnable envelope maps to env (formed inside, matris_env_linear)."""
    return _AtomRefinement.apply(atom, bond, basis, layer, ag, d2u)
