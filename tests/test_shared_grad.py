"""The shared gradient buffer of tensors read by several fused layers (fused.shared_grad):
readers that write their gradient into the accumulator and return None, mixed with plain
torch readers, give autograd's gradient exactly, also under non-reentrant checkpointing
and a second backward.  CPU only: the readers here are toy autograd Functions that use the
accumulator the way the fused Refinements do (first writer stores, later ones add)."""
import torch
import torch.utils.checkpoint

from matris_amd.model import fused


class _ScaleReader(torch.autograd.Function):
    """y = k * x; its x-gradient goes into x's accumulator when there is one."""

    @staticmethod
    def forward(ctx, x, k):
        ctx.acc, ctx.k = fused._acc_of(x), k
        return x * k

    @staticmethod
    def backward(ctx, g):
        out, acc = fused._acc_out(ctx.acc)
        gx = g * ctx.k
        if acc:
            out.add_(gx)  # stands for a kernel's accumulate
            gx = out
        return fused._acc_keep(ctx.acc, gx), None


class _AddReader(torch.autograd.Function):
    """y = x + 1, its gradient handed over with _acc_add (the fallback path)."""

    @staticmethod
    def forward(ctx, x):
        ctx.acc = fused._acc_of(x)
        return x + 1.0

    @staticmethod
    def backward(ctx, g):
        return fused._acc_add(ctx.acc, g.clone())


def _block(x):
    s = fused.shared_grad(x)
    return (_ScaleReader.apply(s, 3.0) ** 2).sum() + _AddReader.apply(s).pow(3).sum() + (s * 7).sum()


def _plain(x):
    return ((x * 3.0) ** 2).sum() + (x + 1.0).pow(3).sum() + (x * 7).sum()


def test_accumulated_readers_match_autograd():
    torch.manual_seed(0)
    x = torch.randn(5, 4, dtype=torch.float64, requires_grad=True)
    g_ref, = torch.autograd.grad(_plain(x * 2), x)
    g, = torch.autograd.grad(_block(x * 2), x)
    assert torch.allclose(g, g_ref, rtol=1e-14, atol=0)


def test_only_accumulating_readers():
    x = torch.randn(6, dtype=torch.float64, requires_grad=True)
    s = fused.shared_grad(x * 1.5)
    y = _ScaleReader.apply(s, 2.0).sum() + _ScaleReader.apply(s, -5.0).pow(2).sum()
    g, = torch.autograd.grad(y, x)
    x2 = x.detach().clone().requires_grad_(True)
    g_ref, = torch.autograd.grad((2.0 * 1.5 * x2).sum() + (-5.0 * 1.5 * x2).pow(2).sum(), x2)
    assert torch.allclose(g, g_ref, rtol=1e-14, atol=0)


def test_under_checkpoint_and_second_backward():
    torch.manual_seed(1)
    x = torch.randn(3, 7, dtype=torch.float64, requires_grad=True)
    g_ref, = torch.autograd.grad(_plain(x.exp()), x)
    y = torch.utils.checkpoint.checkpoint(_block, x.exp(), use_reentrant=False)
    g1, = torch.autograd.grad(y, x, retain_graph=True)
    g2, = torch.autograd.grad(y, x)  # the accumulator was emptied by the first backward
    assert torch.allclose(g1, g_ref, rtol=1e-14, atol=0)
    assert torch.allclose(g2, g_ref, rtol=1e-14, atol=0)


def test_no_grad_returns_the_tensor_itself():
    x = torch.randn(3, requires_grad=True)
    with torch.no_grad():
        assert fused.shared_grad(x) is x
    y = torch.randn(3)
    assert fused.shared_grad(y) is y
