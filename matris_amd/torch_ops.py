"""PyTorch dispatcher ops over libmatris_hip.so (torch.library custom ops).

Importing this module registers two op namespaces with schemas, shape ("fake") functions
for tracing, and autograd formulas where the op is differentiable:

``matris_op`` -- the reference's own torch op library (matris/model/op/src/RegisterOp.cpp:
9-13, Opdefine.h:7-10), same names, arguments and results, on the HIP kernels of
csrc/silu.hip (the arithmetic of op/fused_silu_op.py:5-28):

    fuse_silu_bwd(Tensor dgrad, Tensor input) -> Tensor
    fuse_silu_grad_bwd(Tensor grad_grad_input, Tensor grad_output, Tensor input) -> Tensor[]

``fused_silu(x)`` is the reference's FusedSiLU entry point (fused_silu_op.py:31-89): SiLU
whose first and second derivatives run through those two ops.

``matris_hip`` -- the path's kernels as ops (the boundary of the hot path, one op per
C-ABI launcher family): segment sums and gathers over CSR groupings (functions.py:129-
160), the fused segment attention (interaction_block.py:113-134 with functions.py:97-127),
the gated MLP (functions.py:245-311), the bias-free FFN (functions.py:198-205), the
attention projection pair (interaction_block.py:33-38) and the periodic radius graph
(converter.py:57-60).  Weights are plain tensors in their module layout; their MFMA
packing is cached per (data pointer, version).

Every op runs on the current HIP stream and allocates its outputs from torch's caching
allocator; only ``csr_build`` (a key range check) and ``radius_graph`` (the edge count)
read anything back to the host, so the others can be captured in a HIP graph.  Inputs
are checked (device, dtype, contiguity, shape) and a failed check raises RuntimeError;
the ops have no CPU kernels (a CPU tensor raises NotImplementedError from the
dispatcher).  The GEMM ops run in the arithmetic that ops.set_mma_precision selects.
"""
from collections import OrderedDict
from typing import Optional, Sequence

import torch
from torch import Tensor

from . import _lib
from .model import ops

D = ops.D


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _f32(name: str, t: Tensor, cols: int | None = None) -> None:
    _check(t.is_cuda, f"{name} must be a ROCm device tensor")
    _check(t.dtype == torch.float32, f"{name} must be float32, got {t.dtype}")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    if cols is not None:
        _check(t.dim() == 2 and t.shape[1] == cols, f"{name} must be [*, {cols}], got {tuple(t.shape)}")


def _i32(name: str, t: Tensor, n: int | None = None) -> None:
    _check(t.is_cuda, f"{name} must be a ROCm device tensor")
    _check(t.dtype == torch.int32 and t.is_contiguous(), f"{name} must be contiguous int32")
    if n is not None:
        _check(t.numel() == n, f"{name} must have {n} entries, got {t.numel()}")


def _grouping(key: Tensor, rowptr: Tensor, perm: Optional[Tensor]) -> ops.Grouping:
    return ops.Grouping(key, rowptr, perm, rowptr.numel() - 1)


# ------------------------------------------------------------------------------------
# weight packs, cached by the weights' identity
# ------------------------------------------------------------------------------------
_PACKS = OrderedDict()
_MAX_PACKS = 64


def _cached(kind: str, tensors, make):
    key = (kind,) + tuple((t.data_ptr(), t._version, tuple(t.shape)) if t is not None else None for t in tensors)
    pack = _PACKS.get(key)
    if pack is None:
        pack = make()
        _PACKS[key] = pack
        if len(_PACKS) > _MAX_PACKS:
            _PACKS.popitem(last=False)
    else:
        _PACKS.move_to_end(key)
    return pack


def _gmlp_pack(w1, b1, w2, b2, norm_c, norm_g, eps):
    _f32("w1", w1)
    _check(w1.dim() == 2 and w1.shape[0] == 256 and w1.shape[1] % D == 0 and 0 < w1.shape[1] <= 4 * D,
           f"w1 must be [256, 128 k] with k in 1..4, got {tuple(w1.shape)}")
    _f32("w2", w2, D)
    _check(w2.shape[0] == 256, f"w2 must be [256, 128], got {tuple(w2.shape)}")
    for name, t, n in (("b1", b1, 256), ("b2", b2, 256), ("norm_c", norm_c, D), ("norm_g", norm_g, D)):
        if t is not None:
            _f32(name, t)
            _check(t.numel() == n, f"{name} must have {n} entries")
    return _cached("gmlp", (w1, b1, w2, b2, norm_c, norm_g),
                   lambda: ops.GmlpPack().get_tensors(w1, b1, w2, b2, norm_c, norm_g, eps)).get_tensors(
        w1, b1, w2, b2, norm_c, norm_g, eps)


def _pair_pack(w0, w1):
    for name, t in (("w0", w0), ("w1", w1)):
        _f32(name, t, D)
        _check(t.shape[0] == D, f"{name} must be [128, 128], got {tuple(t.shape)}")
    return _cached("pair", (w0, w1), lambda: ops._WeightPack().get(w0, w1)).get(w0, w1)


def _mode() -> int:
    return ops._MMA["mode"]


# ------------------------------------------------------------------------------------
# matris_op: the reference's SiLU derivative ops
# ------------------------------------------------------------------------------------
@torch.library.custom_op("matris_op::fuse_silu_bwd", mutates_args=(), device_types="cuda")
def fuse_silu_bwd(dgrad: Tensor, input: Tensor) -> Tensor:
    """dgrad * SiLU'(input) (Opdefine.h:7; fused_silu_op.py:5-14)."""
    _f32("dgrad", dgrad)
    _f32("input", input)
    _check(dgrad.shape == input.shape, "dgrad and input must have the same shape")
    out = torch.empty_like(input)
    _lib.check(_lib.load().matris_silu_bwd(input.numel(), ops._p(dgrad), ops._p(input), ops._p(out), ops._stream()),
               "matris_silu_bwd")
    return out


@fuse_silu_bwd.register_fake
def _(dgrad, input):
    return torch.empty_like(input)


@torch.library.custom_op("matris_op::fuse_silu_grad_bwd", mutates_args=(), device_types="cuda")
def fuse_silu_grad_bwd(grad_grad_input: Tensor, grad_output: Tensor, input: Tensor) -> list[Tensor]:
    """[grad_grad_input * SiLU'(input), grad_grad_input * grad_output * SiLU''(input)]
    (Opdefine.h:8-10; fused_silu_op.py:17-28)."""
    for name, t in (("grad_grad_input", grad_grad_input), ("grad_output", grad_output), ("input", input)):
        _f32(name, t)
        _check(t.shape == input.shape, f"{name} must have input's shape")
    ggo, gx = torch.empty_like(input), torch.empty_like(input)
    _lib.check(_lib.load().matris_silu_grad_bwd(input.numel(), ops._p(grad_grad_input), ops._p(grad_output),
                                                ops._p(input), ops._p(ggo), ops._p(gx), ops._stream()),
               "matris_silu_grad_bwd")
    return [ggo, gx]


@fuse_silu_grad_bwd.register_fake
def _(grad_grad_input, grad_output, input):
    return [torch.empty_like(input), torch.empty_like(input)]


def _silu_bwd_setup(ctx, inputs, output):
    dgrad, x = inputs
    ctx.save_for_backward(dgrad, x)


def _silu_bwd_backward(ctx, grad_grad_input):
    dgrad, x = ctx.saved_tensors
    ggo, gx = torch.ops.matris_op.fuse_silu_grad_bwd(grad_grad_input.contiguous(), dgrad, x)
    return ggo, gx


torch.library.register_autograd("matris_op::fuse_silu_bwd", _silu_bwd_backward, setup_context=_silu_bwd_setup)


class _FusedSiLU(torch.autograd.Function):
    """SiLU forward, backward through matris_op.fuse_silu_bwd (whose own derivative is
    fuse_silu_grad_bwd): fused_silu_op.py:31-89."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return torch.nn.functional.silu(x)

    @staticmethod
    def backward(ctx, grad_output):
        (x,) = ctx.saved_tensors
        return torch.ops.matris_op.fuse_silu_bwd(grad_output.contiguous(), x)


def fused_silu(x: Tensor) -> Tensor:
    """The reference's fused_silu (fused_silu_op.py:84-89) on the device; no CPU path."""
    _check(x.is_cuda, "fused_silu runs on the ROCm device only (no CPU fallback)")
    return _FusedSiLU.apply(x)


# ------------------------------------------------------------------------------------
# matris_hip: segment sums, gathers, CSR groupings
# ------------------------------------------------------------------------------------
@torch.library.custom_op("matris_hip::csr_build", mutates_args=(), device_types="cuda")
def csr_build(key: Tensor, n_seg: int) -> tuple[Tensor, Tensor]:
    """(rowptr int32 [n_seg+1], perm int32 [R]) of the stable CSR grouping of rows by key
    (matris_csr_build); a key outside [0, n_seg) raises.  Reads the check to the host."""
    _i32("key", key)
    grp = ops.Grouping.build(key, int(n_seg))
    return grp.rowptr, grp.perm.clone()


@csr_build.register_fake
def _(key, n_seg):
    return key.new_empty(n_seg + 1), key.new_empty(key.numel())


@torch.library.custom_op("matris_hip::seg_sum", mutates_args=(), device_types="cuda")
def seg_sum(x: Tensor, key: Tensor, rowptr: Tensor, perm: Optional[Tensor]) -> Tensor:
    """out[s] = sum of x's rows of segment s (rows perm[rowptr[s]:rowptr[s+1]], perm None =
    rows ascending by key): aggregate / index_add_ (functions.py:129-160), fixed order."""
    _f32("x", x, D)
    _i32("key", key, x.shape[0])
    _i32("rowptr", rowptr)
    if perm is not None:
        _i32("perm", perm, x.shape[0])
    with ops.exact_rows():
        return ops.seg_sum_raw(x, _grouping(key, rowptr, perm))


@seg_sum.register_fake
def _(x, key, rowptr, perm):
    return x.new_empty(rowptr.shape[0] - 1, D)


def _seg_sum_setup(ctx, inputs, output):
    ctx.key = inputs[1]


def _seg_sum_backward(ctx, g):
    return torch.ops.matris_hip.gather_rows(g.contiguous(), ctx.key), None, None, None


torch.library.register_autograd("matris_hip::seg_sum", _seg_sum_backward, setup_context=_seg_sum_setup)


@torch.library.custom_op("matris_hip::gather_rows", mutates_args=(), device_types="cuda")
def gather_rows(src: Tensor, idx: Tensor) -> Tensor:
    """src[idx] (index_select, interaction_block.py:96-100).  Not differentiable as an op
    (its gradient needs idx's CSR grouping: use gather)."""
    _f32("src", src, D)
    _i32("idx", idx)
    with ops.exact_rows():
        return ops.gather_raw(src, idx)


@gather_rows.register_fake
def _(src, idx):
    return src.new_empty(idx.numel(), D)


@torch.library.custom_op("matris_hip::gather", mutates_args=(), device_types="cuda")
def gather(src: Tensor, idx: Tensor, idx_rowptr: Tensor, idx_perm: Optional[Tensor]) -> Tensor:
    """src[idx] with its gradient as the fixed-order segment sum over idx's CSR grouping
    (idx_rowptr [src rows + 1], idx_perm as csr_build returns)."""
    _i32("idx_rowptr", idx_rowptr, src.shape[0] + 1)
    return gather_rows(src, idx)


@gather.register_fake
def _(src, idx, idx_rowptr, idx_perm):
    return src.new_empty(idx.numel(), D)


def _gather_setup(ctx, inputs, output):
    ctx.idx, ctx.rowptr, ctx.perm = inputs[1], inputs[2], inputs[3]


def _gather_backward(ctx, g):
    return torch.ops.matris_hip.seg_sum(g.contiguous(), ctx.idx, ctx.rowptr, ctx.perm), None, None, None


torch.library.register_autograd("matris_hip::gather", _gather_backward, setup_context=_gather_setup)


# ------------------------------------------------------------------------------------
# matris_hip: segment attention
# ------------------------------------------------------------------------------------
@torch.library.custom_op("matris_hip::line_attn_fwd", mutates_args=(), device_types="cuda")
def line_attn_fwd(alpha_t: Tensor, alpha_s: Tensor, e: Tensor, tgt_key: Tensor, tgt_rowptr: Tensor,
                  tgt_perm: Optional[Tensor], src_key: Tensor, src_rowptr: Tensor,
                  src_perm: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(y_t, y_s, lse_t, lse_s): Dimwise_softmax of alpha_t by target and of alpha_s by
    source (functions.py:97-127), each times e and summed per segment
    (interaction_block.py:113-134); lse = per-segment, per-column log-sum-exp (rows of
    empty segments: y = 0, lse unwritten)."""
    R = e.shape[0]
    for name, t in (("alpha_t", alpha_t), ("alpha_s", alpha_s), ("e", e)):
        _f32(name, t, D)
        _check(t.shape[0] == R, f"{name} must have e's rows")
    for name, t in (("tgt_key", tgt_key), ("src_key", src_key)):
        _i32(name, t, R)
    _check(tgt_rowptr.numel() == src_rowptr.numel(), "tgt and src groupings need the same segment count")
    with ops.exact_rows():
        return ops.attn_fwd_raw(alpha_t, alpha_s, e, _grouping(tgt_key, tgt_rowptr, tgt_perm),
                                _grouping(src_key, src_rowptr, src_perm), None)


@line_attn_fwd.register_fake
def _(alpha_t, alpha_s, e, tgt_key, tgt_rowptr, tgt_perm, src_key, src_rowptr, src_perm):
    S = tgt_rowptr.shape[0] - 1
    return tuple(e.new_empty(S, D) for _ in range(4))


@torch.library.custom_op("matris_hip::line_attn_bwd", mutates_args=(), device_types="cuda")
def line_attn_bwd(alpha_t: Tensor, alpha_s: Tensor, e: Tensor, y_t: Tensor, y_s: Tensor, lse_t: Tensor,
                  lse_s: Tensor, g_yt: Tensor, g_ys: Tensor, tgt_key: Tensor, src_key: Tensor,
                  n_seg: int) -> tuple[Tensor, Tensor, Tensor]:
    """(g_alpha_t, g_alpha_s, g_e) per row: the input gradients of line_attn_fwd's y_t, y_s
    for output gradients g_yt, g_ys [n_seg, 128]."""
    R = e.shape[0]
    for name, t in (("alpha_t", alpha_t), ("alpha_s", alpha_s), ("e", e)):
        _f32(name, t, D)
    for name, t in (("y_t", y_t), ("y_s", y_s), ("lse_t", lse_t), ("lse_s", lse_s), ("g_yt", g_yt), ("g_ys", g_ys)):
        _f32(name, t, D)
        _check(t.shape[0] == n_seg, f"{name} must have n_seg rows")
    _i32("tgt_key", tgt_key, R)
    _i32("src_key", src_key, R)
    dummy = torch.empty(0, dtype=torch.int32, device=e.device)
    tgt, src = ops.Grouping(tgt_key, dummy, None, int(n_seg)), ops.Grouping(src_key, dummy, None, int(n_seg))
    with ops.exact_rows():
        return ops.attn_bwd_raw(alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s, g_yt, g_ys, tgt, src, None)


@line_attn_bwd.register_fake
def _(alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s, g_yt, g_ys, tgt_key, src_key, n_seg):
    return tuple(e.new_empty(e.shape[0], D) for _ in range(3))


# ------------------------------------------------------------------------------------
# matris_hip: gated MLP, FFN, projection pair
# ------------------------------------------------------------------------------------
@torch.library.custom_op("matris_hip::gated_mlp_fwd", mutates_args=(), device_types="cuda")
def gated_mlp_fwd(srcs: Sequence[Tensor], idxs: Sequence[Optional[Tensor]], n_rows: int, w1: Tensor,
                  b1: Optional[Tensor], w2: Tensor, b2: Optional[Tensor], norm_c: Tensor, norm_g: Tensor,
                  eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """(out [n_rows,128], p [n_rows,256], z [n_rows,256]) of GatedMLP with RMSNorm
    (functions.py:245-311) on x = concat_j srcs[j][idxs[j]] (an index None: the source's
    own rows); w1 = [core; gate] layer-1 weights [256, 128 len(srcs)], w2 = [core; gate]
    layer-2 weights [256, 128].  p, z are what gated_mlp_bwd needs."""
    _check(1 <= len(srcs) <= 4 and len(idxs) == len(srcs), "one to four sources, one index (or None) each")
    _check(w1.shape[1] == D * len(srcs), "w1 must have 128 columns per source")
    for j, (s, i) in enumerate(zip(srcs, idxs)):
        _f32(f"srcs[{j}]", s, D)
        if i is None:
            _check(s.shape[0] == n_rows, f"srcs[{j}] without an index must have n_rows rows")
        else:
            _i32(f"idxs[{j}]", i, n_rows)
    pack = _gmlp_pack(w1, b1, w2, b2, norm_c, norm_g, eps)
    with ops.exact_rows():
        out, p, z, _ = ops.gmlp_fwd_raw(pack, list(srcs), list(idxs), int(n_rows), _mode())
    return out, p, z


@gated_mlp_fwd.register_fake
def _(srcs, idxs, n_rows, w1, b1, w2, b2, norm_c, norm_g, eps):
    s = srcs[0]
    return s.new_empty(n_rows, D), s.new_empty(n_rows, 256), s.new_empty(n_rows, 256)


@torch.library.custom_op("matris_hip::gated_mlp_bwd", mutates_args=(), device_types="cuda")
def gated_mlp_bwd(g_out: Tensor, p: Tensor, z: Tensor, w1: Tensor, b1: Optional[Tensor], w2: Tensor,
                  b2: Optional[Tensor], norm_c: Tensor, norm_g: Tensor, eps: float) -> Tensor:
    """g_x [M, K]: the gradient of gated_mlp_fwd's out with respect to its concatenated
    input x, from the saved p, z (per-source scatters are the caller's segment sums)."""
    M = p.shape[0]
    _f32("g_out", g_out, D)
    _f32("p", p, 256)
    _f32("z", z, 256)
    _check(g_out.shape[0] == M and z.shape[0] == M, "g_out, p and z must have the same rows")
    pack = _gmlp_pack(w1, b1, w2, b2, norm_c, norm_g, eps)
    with ops.exact_rows():
        return ops.gmlp_bwd_raw(pack, g_out, p, z, int(w1.shape[1]), _mode())


@gated_mlp_bwd.register_fake
def _(g_out, p, z, w1, b1, w2, b2, norm_c, norm_g, eps):
    return g_out.new_empty(p.shape[0], w1.shape[1])


@torch.library.custom_op("matris_hip::ffn_fwd", mutates_args=(), device_types="cuda")
def ffn_fwd(x: Tensor, w1: Tensor, w2: Tensor) -> tuple[Tensor, Tensor]:
    """(out, p): MLP(hidden=128, bias=False) = SiLU(x W1^T) W2^T (functions.py:198-205),
    p = x W1^T saved for ffn_bwd; weights [128, 128] as in nn.Linear."""
    _f32("x", x, D)
    pack = _pair_pack(w1, w2)
    with ops.exact_rows():
        return ops.ffn_fwd_raw(pack, x, _mode())


@ffn_fwd.register_fake
def _(x, w1, w2):
    return x.new_empty(x.shape[0], D), x.new_empty(x.shape[0], D)


@torch.library.custom_op("matris_hip::ffn_bwd", mutates_args=(), device_types="cuda")
def ffn_bwd(g: Tensor, p: Tensor, w1: Tensor, w2: Tensor) -> Tensor:
    """g_x of ffn_fwd for the output gradient g."""
    _f32("g", g, D)
    _f32("p", p, D)
    _check(g.shape[0] == p.shape[0], "g and p must have the same rows")
    pack = _pair_pack(w1, w2)
    with ops.exact_rows():
        return ops.ffn_bwd_raw(pack, g, p, _mode())


@ffn_bwd.register_fake
def _(g, p, w1, w2):
    return g.new_empty(g.shape[0], D)


@torch.library.custom_op("matris_hip::pair_fwd", mutates_args=(), device_types="cuda")
def pair_fwd(x: Tensor, w_s: Tensor, w_t: Tensor) -> tuple[Tensor, Tensor]:
    """(x W_s^T, x W_t^T) from one read of x: source_weight_linear and
    target_weight_linear (interaction_block.py:33-38, 110-111)."""
    _f32("x", x, D)
    pack = _pair_pack(w_s, w_t)
    with ops.exact_rows():
        return ops.pair_fwd_raw(pack, x, _mode())


@pair_fwd.register_fake
def _(x, w_s, w_t):
    return x.new_empty(x.shape[0], D), x.new_empty(x.shape[0], D)


@torch.library.custom_op("matris_hip::pair_bwd", mutates_args=(), device_types="cuda")
def pair_bwd(g_s: Tensor, g_t: Tensor, w_s: Tensor, w_t: Tensor) -> Tensor:
    """g_s W_s + g_t W_t: the input gradient of pair_fwd."""
    _f32("g_s", g_s, D)
    _f32("g_t", g_t, D)
    _check(g_s.shape[0] == g_t.shape[0], "g_s and g_t must have the same rows")
    pack = _pair_pack(w_s, w_t)
    with ops.exact_rows():
        return ops.pair_bwd_raw(pack, g_s, g_t, _mode())


@pair_bwd.register_fake
def _(g_s, g_t, w_s, w_t):
    return g_s.new_empty(g_s.shape[0], D)


# ------------------------------------------------------------------------------------
# matris_hip: graph
# ------------------------------------------------------------------------------------
@torch.library.custom_op("matris_hip::radius_graph", mutates_args=(), device_types="cuda")
def radius_graph(frac: Tensor, lattice: Tensor, cutoff: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(center, neighbor int32 [E], image int32 [E,3], dist fp64 [E], row_ptr int64 [n+1]):
    every periodic neighbour within cutoff of the fp64 fractional coordinates frac [n,3]
    (device) in the lattice rows lattice [3,3] (any device), in the canonical order
    (center, then neighbour, then image) -- the neighbour list of converter.py:57-60.
    Reads the edge count to the host."""
    _check(frac.is_cuda and frac.dtype == torch.float64 and frac.dim() == 2 and frac.shape[1] == 3,
           "frac must be a fp64 [n, 3] device tensor")
    _check(lattice.dtype == torch.float64 and tuple(lattice.shape) == (3, 3), "lattice must be fp64 [3, 3]")
    from .graph.converter import radius_graph_device
    c, nb, im, d, rp, _ = radius_graph_device(frac, lattice.detach().cpu().numpy(), float(cutoff))
    return c.clone(), nb.clone(), im.clone(), d.clone(), rp


@radius_graph.register_fake
def _(frac, lattice, cutoff):
    ctx = torch.library.get_ctx()
    E = ctx.new_dynamic_size()
    n = frac.shape[0]
    return (frac.new_empty(E, dtype=torch.int32), frac.new_empty(E, dtype=torch.int32),
            frac.new_empty(E, 3, dtype=torch.int32), frac.new_empty(E, dtype=torch.float64),
            frac.new_empty(n + 1, dtype=torch.int64))


OPS = {
    "matris_op": ("fuse_silu_bwd", "fuse_silu_grad_bwd"),
    "matris_hip": ("csr_build", "seg_sum", "gather_rows", "gather", "line_attn_fwd", "line_attn_bwd",
                   "gated_mlp_fwd", "gated_mlp_bwd", "ffn_fwd", "ffn_bwd", "pair_fwd", "pair_bwd", "radius_graph"),
}
