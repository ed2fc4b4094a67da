"""GPU parity of the chunked tied-head cross-entropy (chunked_lm_loss.py:5-84).

The HIP cross-entropy rows (``mogt_lm_ce_fwd`` / ``mogt_lm_ce_bwd`` through
``mogt_amd.ops``) against the float64 oracle (oracle/lm_loss_oracle.py) on the
same logits, including unaligned rows (strided views), odd vocabularies,
ignored (-100) and out-of-range labels; then chunked_linear_cross_entropy end to
end (loss and both gradients) against the float64 chunked oracle, and the
model's chunked loss paths (model_mogt.py:326-380) against its unchunked loss.
Bars: the rows compute in fp32 from exactly representable inputs, <= 1e-5
normwise; the end-to-end path adds fp32 GEMMs, <= 1e-4; bf16 hidden states
(gradient returned in bf16) <= 2e-2."""
import numpy as np
import pytest
import torch

from conftest import announce, rel_err, to_np
from oracle import lm_loss_oracle as lo

pytestmark = pytest.mark.gpu

ROW_TOL = 1e-5
E2E_TOL = 1e-4
BF16_TOL = 2e-2


def _logits(rows, vocab, dtype, gpu, seed, pad=0):
    g = torch.Generator().manual_seed(seed)
    full = torch.randn(rows, vocab + pad, generator=g) * 4.0
    x = full.to(gpu).to(dtype)
    return x[:, pad // 2: pad // 2 + vocab] if pad else x


def _labels(rows, vocab, gpu, seed, ignore_every=0):
    g = torch.Generator().manual_seed(seed + 1)
    lab = torch.randint(0, vocab, (rows,), generator=g)
    if ignore_every:
        lab[::ignore_every] = -100
    return lab.to(gpu)


CASES = [(1, 1, torch.float32, 0), (3, 7, torch.float32, 0), (64, 129, torch.float32, 3),
         (257, 32000, torch.float32, 0), (33, 50257, torch.float32, 2), (40, 50257, torch.bfloat16, 5),
         (100, 32000, torch.bfloat16, 0), (5, 4095, torch.bfloat16, 3)]


@pytest.mark.parametrize("rows,vocab,dtype,pad", CASES)
def test_ce_rows_forward(gpu, rows, vocab, dtype, pad):
    announce(f"ce rows fwd rows={rows} vocab={vocab} {dtype} pad={pad}")
    from mogt_amd import ops

    x = _logits(rows, vocab, dtype, gpu, seed=rows + vocab, pad=pad)
    lab = _labels(rows, vocab, gpu, seed=rows, ignore_every=4 if rows > 4 else 0)
    loss, lse = ops.lm_ce_forward(x, lab)
    torch.cuda.synchronize()
    ref_loss, ref_lse = lo.ce_rows(to_np(x), lab.cpu().numpy())
    assert loss.dtype == torch.float32 and lse.shape == (rows,)
    assert rel_err(to_np(lse), ref_lse) <= ROW_TOL
    assert rel_err(to_np(loss), ref_loss) <= ROW_TOL
    assert float(loss[lab == -100].abs().sum()) == 0.0


@pytest.mark.parametrize("rows,vocab,dtype,pad", CASES)
def test_ce_rows_backward_in_place(gpu, rows, vocab, dtype, pad):
    announce(f"ce rows bwd rows={rows} vocab={vocab} {dtype} pad={pad}")
    from mogt_amd import ops

    x = _logits(rows, vocab, dtype, gpu, seed=rows * 3 + vocab, pad=pad)
    lab = _labels(rows, vocab, gpu, seed=rows + 7, ignore_every=3 if rows > 3 else 0)
    x_np = to_np(x)
    _, lse = ops.lm_ce_forward(x, lab)
    scale = torch.tensor([0.37], device=gpu)
    out = ops.lm_ce_backward_(x, lab, lse, scale)
    torch.cuda.synchronize()
    assert out.data_ptr() == x.data_ptr()
    ref = lo.ce_rows_grad(x_np, lab.cpu().numpy(), 0.37)
    tol = ROW_TOL if dtype == torch.float32 else 4e-3   # the gradient itself is stored in bf16
    assert rel_err(to_np(x), ref) <= tol
    assert float(x[lab == -100].float().abs().sum()) == 0.0


def test_ce_rows_bad_label_is_nan(gpu):
    from mogt_amd import ops

    x = _logits(4, 50, torch.float32, gpu, seed=1)
    lab = torch.tensor([3, 50, -1, -100], device=gpu)
    loss, lse = ops.lm_ce_forward(x, lab)
    ops.lm_ce_backward_(x, lab, lse, torch.ones(1, device=gpu))
    torch.cuda.synchronize()
    l = loss.cpu()
    assert torch.isfinite(l[0]) and torch.isnan(l[1]) and torch.isnan(l[2]) and l[3] == 0
    assert torch.isnan(x[1]).all() and torch.isnan(x[2]).all() and (x[3] == 0).all()
    assert torch.isfinite(x[0]).all()


def test_ce_rows_argument_errors(gpu):
    from mogt_amd import ops

    x = torch.zeros(4, 10, device=gpu)
    with pytest.raises(ValueError):
        ops.lm_ce_forward(x, torch.zeros(4, dtype=torch.int32, device=gpu))
    with pytest.raises(ValueError):
        ops.lm_ce_forward(x.t(), torch.zeros(10, dtype=torch.int64, device=gpu))
    with pytest.raises(ValueError):
        ops.lm_ce_backward_(x, torch.zeros(4, dtype=torch.int64, device=gpu), torch.zeros(4, device=gpu),
                            torch.ones(2, device=gpu))


@pytest.mark.parametrize("chunk", [1, 64, 333, 10000])
def test_chunked_linear_ce_matches_oracle(gpu, chunk):
    announce(f"chunked linear CE chunk={chunk}")
    from mogt_amd.chunked_lm_loss import chunked_linear_cross_entropy

    g = torch.Generator().manual_seed(chunk)
    B, L, D, V = 2, 300, 64, 1000
    h = torch.randn(B, L, D, generator=g)
    w = torch.randn(V, D, generator=g) * 0.3
    lab = torch.randint(0, V, (B, L), generator=g)
    lab[1, ::17] = -100
    ht = h.to(gpu).requires_grad_()
    wt = w.to(gpu).requires_grad_()
    loss = chunked_linear_cross_entropy(ht, wt, lab.to(gpu), chunk_size=chunk)
    (loss * 2.5).backward()
    torch.cuda.synchronize()
    ref_loss, ref_gh, ref_gw = lo.chunked_linear_ce(h.numpy(), w.numpy(), lab.numpy(), chunk, grad_output=2.5)
    assert abs(float(loss.detach()) - ref_loss) <= E2E_TOL * abs(ref_loss)
    assert rel_err(to_np(ht.grad), ref_gh) <= E2E_TOL
    assert rel_err(to_np(wt.grad), ref_gw) <= E2E_TOL


def test_chunked_linear_ce_bf16_hidden(gpu):
    announce("chunked linear CE bf16 hidden")
    from mogt_amd.chunked_lm_loss import chunked_linear_cross_entropy

    g = torch.Generator().manual_seed(5)
    B, L, D, V = 1, 512, 128, 4096
    h = torch.randn(B, L, D, generator=g).bfloat16()
    w = torch.randn(V, D, generator=g) * 0.1
    lab = torch.randint(0, V, (B, L), generator=g)
    ht = h.to(gpu).requires_grad_()
    wt = w.to(gpu).requires_grad_()
    loss = chunked_linear_cross_entropy(ht, wt, lab.to(gpu), chunk_size=200)
    loss.backward()
    torch.cuda.synchronize()
    ref_loss, ref_gh, ref_gw = lo.chunked_linear_ce(h.float().numpy(), w.numpy(), lab.numpy(), 200)
    assert ht.grad.dtype == torch.bfloat16 and wt.grad.dtype == torch.float32
    assert abs(float(loss.detach()) - ref_loss) <= E2E_TOL * abs(ref_loss)
    assert rel_err(to_np(ht.grad), ref_gh) <= BF16_TOL
    assert rel_err(to_np(wt.grad), ref_gw) <= E2E_TOL


def test_chunked_linear_ce_validation(gpu):
    from mogt_amd.chunked_lm_loss import chunked_linear_cross_entropy

    h = torch.zeros(1, 4, 8, device=gpu)
    w = torch.zeros(10, 8, device=gpu)
    lab = torch.zeros(1, 4, dtype=torch.int64, device=gpu)
    for args, msg in [((h[0], w, lab[0]), "hidden_states"), ((h, w, lab[:, :3]), "labels"),
                      ((h, w[:, :7], lab), "weight")]:
        with pytest.raises(ValueError, match=msg):
            chunked_linear_cross_entropy(*args, chunk_size=2)
    with pytest.raises(ValueError, match="chunk_size"):
        chunked_linear_cross_entropy(h, w, lab, chunk_size=0)


def test_model_chunked_loss_paths(gpu):
    """MOGTForCausalLM.forward (model_mogt.py:350-380): unchunked loss, chunked
    loss with logits, chunked linear CE without logits -- same loss, and the
    linear-CE path's gradients equal the unchunked ones."""
    announce("model chunked loss paths")
    from mogt_amd.model_mogt import MOGTForCausalLM

    torch.manual_seed(3)
    model = MOGTForCausalLM(vocab_size=257, d_model=64, num_layers=1, r=16).to(gpu)
    ids = torch.randint(0, 257, (1, 200), device=gpu)
    labels = torch.randint(0, 257, (1, 200), device=gpu)
    _, l0 = model(ids, labels=labels)
    l0.backward()
    g0 = {k: p.grad.clone() for k, p in model.named_parameters() if p.grad is not None}
    model.zero_grad()
    logits1, l1 = model(ids, labels=labels, loss_chunk_size=64)
    model.zero_grad()
    logits2, l2 = model(ids, labels=labels, return_logits=False, loss_chunk_size=64)
    l2.backward()
    torch.cuda.synchronize()
    assert logits1.shape == (1, 200, 257) and logits2 is None
    l0, l1, l2 = (float(v.detach()) for v in (l0, l1, l2))
    assert abs(l1 - l0) <= 1e-5 * abs(l0)
    assert abs(l2 - l0) <= 1e-5 * abs(l0)
    for k, p in model.named_parameters():
        if k in g0:
            assert rel_err(to_np(p.grad), to_np(g0[k])) <= E2E_TOL, k
