"""The token embedding's backward (csrc/embedding_bwd.hip) against float64.

dW[v] is the sum of the gradient rows of every position holding token v
(what torch's embedding backward computes for MOGTModel's nn.Embedding,
model_mogt.py:262, 270).  Bar: fp32 normwise max relative error <= 1e-4; the
kernel sums in position order, so two runs agree bit for bit."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import announce, rel_err, to_np

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4


def _ref(grad: torch.Tensor, ids: torch.Tensor, vocab: int) -> np.ndarray:
    g = grad.detach().double().cpu().reshape(-1, grad.shape[-1])
    out = torch.zeros(vocab, g.shape[1], dtype=torch.float64)
    out.index_add_(0, ids.cpu().reshape(-1).long(), g)
    return out.numpy()


def _ids(kind: str, n: int, vocab: int, gen: torch.Generator) -> torch.Tensor:
    if kind == "uniform":
        return torch.randint(0, vocab, (n,), generator=gen)
    if kind == "skewed":   # a few very frequent tokens: runs spanning many 16-position blocks
        hot = torch.randint(0, 4, (n,), generator=gen)
        cold = torch.randint(0, vocab, (n,), generator=gen)
        return torch.where(torch.rand(n, generator=gen) < 0.7, hot, cold)
    if kind == "constant":
        return torch.full((n,), vocab - 1, dtype=torch.int64)
    if kind == "sorted_desc":
        return torch.arange(n, dtype=torch.int64).flip(0) % vocab
    raise ValueError(kind)


@pytest.mark.parametrize("kind,n,vocab,D,dt", [
    ("uniform", 32768, 32000, 768, torch.float32),
    ("uniform", 1000, 50, 768, torch.float32),
    ("skewed", 5003, 300, 768, torch.float32),
    ("constant", 1001, 7, 64, torch.float32),
    ("sorted_desc", 77, 5, 4, torch.float32),
    ("uniform", 1, 10, 4096, torch.float32),
    ("skewed", 4099, 1000, 768, torch.bfloat16),
])
def test_embedding_backward_matches_float64(gpu, kind, n, vocab, D, dt):
    announce(f"embedding backward {kind} n={n} V={vocab} D={D} {dt}")
    from mogt_amd import ops

    gen = torch.Generator().manual_seed(n + vocab + D)
    ids = _ids(kind, n, vocab, gen)
    grad = torch.randn(n, D, generator=gen).to(dt)
    dw = torch.ops.mogt.embedding_bwd(grad.to(gpu), ids.to(gpu), vocab)
    dw2 = torch.ops.mogt.embedding_bwd(grad.to(gpu), ids.to(gpu), vocab)
    torch.cuda.synchronize()
    assert dw.shape == (vocab, D) and dw.dtype == torch.float32
    assert rel_err(to_np(dw), _ref(grad, ids, vocab)) <= FP32_TOL
    assert torch.equal(dw, dw2), "two runs differ"


@pytest.mark.parametrize("n,n2,vocab,D,dt", [(32768, 1, 32000, 768, torch.float32), (1000, 7, 50, 768, torch.float32),
                                             (300, 300, 20, 64, torch.bfloat16), (5, 0, 9, 4, torch.float32)])
def test_embedding_backward_two_sources(gpu, n, n2, vocab, D, dt):
    """A second lookup into the same table (the prefix-condition rows): one
    table holds both lookups' gradients, against float64."""
    announce(f"embedding backward two sources n={n}+{n2} V={vocab} D={D} {dt}")
    from mogt_amd import ops  # noqa: F401  (registers the ops)

    gen = torch.Generator().manual_seed(n + n2 + vocab)
    ids = torch.randint(0, vocab, (n,), generator=gen)
    ids2 = torch.randint(0, vocab, (n2,), generator=gen)
    grad = torch.randn(n, D, generator=gen).to(dt)
    grad2 = torch.randn(n2, D, generator=gen).to(dt)
    dw = torch.ops.mogt.embedding_bwd(grad.to(gpu), ids.to(gpu), vocab, grad2.to(gpu), ids2.to(gpu))
    dw_again = torch.ops.mogt.embedding_bwd(grad.to(gpu), ids.to(gpu), vocab, grad2.to(gpu), ids2.to(gpu))
    torch.cuda.synchronize()
    ref = _ref(grad, ids, vocab) + _ref(grad2, ids2, vocab)
    assert rel_err(to_np(dw), ref) <= FP32_TOL
    assert torch.equal(dw, dw_again), "two runs differ"


def test_embedding_pair_gradient_matches_torch(gpu):
    """ops.embedding_pair: the same outputs as two lookups through the module,
    and the weight's gradient of both equal to torch's own backward."""
    announce("embedding pair module gradient")
    from mogt_amd import ops

    torch.manual_seed(5)
    emb = torch.nn.Embedding(700, 256).to(gpu)
    ids = torch.randint(0, 700, (2, 3000), device=gpu)
    w1 = torch.randn(2, 3000, 256, device=gpu)
    w2 = torch.randn(2, 256, device=gpu)
    out, out2 = ops.embedding_pair(ids, ids[:, 1], emb)
    ((out * w1).sum() + (out2 * w2).sum()).backward()
    ours = emb.weight.grad.clone()
    emb.weight.grad = None
    r1, r2 = F.embedding(ids, emb.weight), F.embedding(ids[:, 1], emb.weight)
    ((r1 * w1).sum() + (r2 * w2).sum()).backward()
    torch.cuda.synchronize()
    assert torch.equal(out, r1) and torch.equal(out2, r2)
    assert rel_err(to_np(ours), to_np(emb.weight.grad)) <= FP32_TOL


def test_embedding_module_gradient_matches_torch(gpu):
    """ops.embedding on an nn.Embedding: same output as the module, the
    weight's gradient equal to torch's own backward to fp32 rounding."""
    announce("embedding module gradient")
    from mogt_amd import ops

    torch.manual_seed(4)
    emb = torch.nn.Embedding(500, 768).to(gpu)
    ids = torch.randint(0, 500, (2, 3000), device=gpu)
    w = torch.randn(2, 3000, 768, device=gpu)
    out = ops.embedding(ids, emb)
    (out * w).sum().backward()
    ours = emb.weight.grad.clone()
    emb.weight.grad = None
    ref_out = F.embedding(ids, emb.weight)
    (ref_out * w).sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)
    assert rel_err(to_np(ours), to_np(emb.weight.grad)) <= FP32_TOL


def test_embedding_with_padding_index_uses_the_module(gpu):
    from mogt_amd import ops

    emb = torch.nn.Embedding(20, 8, padding_idx=0).to(gpu)
    ids = torch.tensor([[0, 3, 0, 5]], device=gpu)
    out = ops.embedding(ids, emb)
    out.sum().backward()
    torch.cuda.synchronize()
    assert float(emb.weight.grad[0].abs().sum()) == 0.0   # padding row gets no gradient
