"""AtomTypeEmbedding.embed (feature_embed.py:16-39 on atomic_numbers - 1): its remembered
features are returned only for the same atomic-number tensor, unchanged, with unchanged
weights; every other case recomputes them (CPU)."""
import torch

from matris_amd.model.model import AtomTypeEmbedding


def test_embed_equals_forward_and_is_remembered():
    torch.manual_seed(0)
    emb = AtomTypeEmbedding(128)
    z = torch.tensor([29, 29, 8, 1, 94], dtype=torch.int32)
    a = emb.embed(z)
    assert torch.equal(a, emb(z.long() - 1).detach()) and not a.requires_grad
    assert emb.embed(z) is a  # same tensor, same weights: remembered


def test_embed_recomputes_after_any_change():
    torch.manual_seed(1)
    emb = AtomTypeEmbedding(128)
    z = torch.tensor([29, 8, 8, 14], dtype=torch.int32)
    a = emb.embed(z)
    z2 = z.clone()  # equal values, another tensor
    assert emb.embed(z2) is not a and torch.equal(emb.embed(z2), a)
    z2[0] = 26  # edited in place: version counter
    b = emb.embed(z2)
    assert torch.equal(b, emb(z2.long() - 1).detach()) and not torch.equal(b, a)
    with torch.no_grad():
        emb.atom_swish_layer.linear.weight.mul_(2.0)  # weights edited in place
    c = emb.embed(z2)
    assert c is not b and torch.equal(c, emb(z2.long() - 1).detach())
    emb.load_state_dict({k: v.clone() for k, v in AtomTypeEmbedding(128).state_dict().items()})
    d = emb.embed(z2)
    assert d is not c and torch.equal(d, emb(z2.long() - 1).detach())
