"""The torch op library (matris_amd.torch_ops) on the CPU: every op is registered with its
schema, the reference's matris_op ops keep the reference's names, argument types and
results (matris/model/op/src/RegisterOp.cpp:9-13, Opdefine.h:7-10), the shape functions
give the right shapes under FakeTensorMode (no GPU needed), and CPU tensors find no
kernel (there is no CPU fallback)."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import matris_amd.torch_ops as T

SCHEMAS = {
    "matris_op::fuse_silu_bwd": "(Tensor dgrad, Tensor input) -> Tensor",
    "matris_op::fuse_silu_grad_bwd": "(Tensor grad_grad_input, Tensor grad_output, Tensor input) -> Tensor[]",
    "matris_hip::seg_sum": "(Tensor x, Tensor key, Tensor rowptr, Tensor? perm) -> Tensor",
    "matris_hip::gather": "(Tensor src, Tensor idx, Tensor idx_rowptr, Tensor? idx_perm) -> Tensor",
    "matris_hip::gated_mlp_fwd": ("(Tensor[] srcs, Tensor?[] idxs, SymInt n_rows, Tensor w1, Tensor? b1, Tensor w2, "
                                  "Tensor? b2, Tensor norm_c, Tensor norm_g, float eps) -> (Tensor, Tensor, Tensor)"),
}


def _op(qualname):
    ns, name = qualname.split("::")
    return getattr(getattr(torch.ops, ns), name).default


def test_every_op_is_registered():
    for ns, names in T.OPS.items():
        for name in names:
            assert str(_op(f"{ns}::{name}")._schema).startswith(f"{ns}::{name}(")


@pytest.mark.parametrize("qualname", sorted(SCHEMAS))
def test_schemas(qualname):
    assert str(_op(qualname)._schema) == qualname + SCHEMAS[qualname]


def test_shape_functions_under_fake_tensors():
    with FakeTensorMode():
        dev = "cuda"
        R, S, N = 37, 9, 5
        x = torch.empty(R, 128, device=dev)
        key = torch.empty(R, dtype=torch.int32, device=dev)
        rp = torch.empty(S + 1, dtype=torch.int32, device=dev)
        assert torch.ops.matris_hip.seg_sum(x, key, rp, None).shape == (S, 128)
        assert torch.ops.matris_hip.gather(torch.empty(N, 128, device=dev), key,
                                           torch.empty(N + 1, dtype=torch.int32, device=dev), key).shape == (R, 128)
        outs = torch.ops.matris_hip.line_attn_fwd(x, x, x, key, rp, None, key, rp, key)
        assert [tuple(t.shape) for t in outs] == [(S, 128)] * 4
        grads = torch.ops.matris_hip.line_attn_bwd(x, x, x, *([torch.empty(S, 128, device=dev)] * 6), key, key, S)
        assert [tuple(t.shape) for t in grads] == [(R, 128)] * 3
        w1, w2 = torch.empty(256, 384, device=dev), torch.empty(256, 128, device=dev)
        nv = torch.empty(128, device=dev)
        out, p, z = torch.ops.matris_hip.gated_mlp_fwd([x, torch.empty(N, 128, device=dev), x], [None, key, None], R,
                                                       w1, None, w2, None, nv, nv, 1e-5)
        assert (out.shape, p.shape, z.shape) == ((R, 128), (R, 256), (R, 256))
        assert torch.ops.matris_hip.gated_mlp_bwd(out, p, z, w1, None, w2, None, nv, nv, 1e-5).shape == (R, 384)
        w = torch.empty(128, 128, device=dev)
        assert [tuple(t.shape) for t in torch.ops.matris_hip.ffn_fwd(x, w, w)] == [(R, 128)] * 2
        assert [tuple(t.shape) for t in torch.ops.matris_hip.pair_fwd(x, w, w)] == [(R, 128)] * 2
        assert torch.ops.matris_hip.pair_bwd(x, x, w, w).shape == (R, 128)
        assert torch.ops.matris_op.fuse_silu_bwd(x, x).shape == (R, 128)
        assert [tuple(t.shape) for t in torch.ops.matris_op.fuse_silu_grad_bwd(x, x, x)] == [(R, 128)] * 2


def test_cpu_tensors_have_no_kernel():
    x = torch.zeros(3, 128)
    with pytest.raises(NotImplementedError):
        torch.ops.matris_op.fuse_silu_bwd(x, x)
    with pytest.raises(NotImplementedError):
        torch.ops.matris_hip.seg_sum(x, torch.zeros(3, dtype=torch.int32), torch.zeros(2, dtype=torch.int32), None)
    with pytest.raises(RuntimeError):
        T.fused_silu(x)


def test_width_generic_segment_ops_refuse_cpu_tensors():
    """The torch forms that ops.gather / seg_sum / seg_attention take for rows of another
    width than 128 run on the device only, like the kernels (no CPU fallback)."""
    import pytest
    import torch
    from matris_amd.model import ops
    grp = ops.Grouping(torch.zeros(4, dtype=torch.int32), torch.tensor([0, 4], dtype=torch.int32), None, 1)
    x = torch.zeros(4, 64)
    for call in (lambda: ops.gather(x, grp), lambda: ops.seg_sum(x, grp),
                 lambda: ops.seg_attention(x, x, x, grp, grp)):
        with pytest.raises(RuntimeError, match="ROCm device only"):
            call()
