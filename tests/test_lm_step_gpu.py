"""The config-4 step harness on a small model: loss and every parameter
gradient against a torch fp32 autograd restatement of the same network (same
bf16 weights, token-sequential EFLA), and loss going down over a few steps."""
import math

import numpy as np
import pytest
import torch

from helpers import announce, rel_l2

pytestmark = pytest.mark.gpu


def _efla_seq(q, k, v, beta):
    """Mode Q EFLA, token by token in fp32: S += c k (v - S^T k)^T, o = S^T q."""
    B, T, H, K = q.shape
    S = torch.zeros(B, H, K, v.shape[-1], device=q.device)
    outs = []
    for t in range(T):
        kt, vt, qt, bt = k[:, t], v[:, t], q[:, t], beta[:, t]
        lam = (kt * kt).sum(-1)
        c = -torch.expm1(-bt * lam) / lam
        u = (kt.unsqueeze(-2) @ S).squeeze(-2)
        S = S + c[..., None, None] * kt.unsqueeze(-1) * (vt - u).unsqueeze(-2)
        outs.append((qt.unsqueeze(-2) @ S).squeeze(-2))
    return torch.stack(outs, 1)


def _torch_reference(model, tokens, targets):
    cfg = model.cfg
    D, H, dh = cfg.d_model, cfg.n_heads, cfg.head_dim
    HD = H * dh
    B, T = tokens.shape
    params = {n: model.w(n).float().clone().requires_grad_(True) for n in model.offsets}
    x = params["embed"][tokens.long()].view(B * T, D)
    for i in range(cfg.n_layers):
        L = f"l{i}."
        a = torch.nn.functional.layer_norm(x, (D,), params[L + "ln1.w"], params[L + "ln1.b"],
                                           cfg.ln_eps)
        p = a @ params[L + "w_in"]
        q, k, v = (p[:, j * HD:(j + 1) * HD].reshape(B, T, H, dh) for j in range(3))
        beta = torch.sigmoid(p[:, 3 * HD:]).reshape(B, T, H)
        o = _efla_seq(q, k, v, beta).reshape(B * T, HD)
        x = x + o @ params[L + "w_o"]
        a2 = torch.nn.functional.layer_norm(x, (D,), params[L + "ln2.w"], params[L + "ln2.b"],
                                            cfg.ln_eps)
        u = a2 @ params[L + "w_up"] + params[L + "b_up"]
        g = torch.nn.functional.gelu(u, approximate="tanh")
        x = x + g @ params[L + "w_down"] + params[L + "b_down"]
    af = torch.nn.functional.layer_norm(x, (D,), params["lnf.w"], params["lnf.b"], cfg.ln_eps)
    logits = af @ params["head"]
    loss = torch.nn.functional.cross_entropy(logits, targets.reshape(-1).long())
    loss.backward()
    return loss.item(), {n: t.grad for n, t in params.items()}


def _small():
    from ceo_amd.lm_step import LMConfig

    return LMConfig(vocab=256, d_model=128, n_layers=2, n_heads=2, head_dim=64, mlp=512)


@pytest.fixture(params=[0, 1], ids=["mfma", "generic"])
def gemm_backend(request):
    """The step on the library's large-tile GEMM (default) and on its generic
    kernel only, restoring the default after."""
    from ceo_amd._lib import lib

    assert lib().efla_rt_set_gemm_backend(request.param) == 0
    yield request.param
    assert lib().efla_rt_set_gemm_backend(0) == 0


def test_step_gradients_match_autograd(gemm_backend):
    from ceo_amd.lm_step import EflaLM, synthetic_batch

    announce(f"lm step: gradients vs torch autograd (2 layers, d=128, T=128), "
             f"gemm backend {gemm_backend}")
    cfg = _small()
    model = EflaLM(cfg, seed=1)
    # larger weights than the default init so every path carries signal
    model.master.mul_(4.0)
    model.weights.copy_(model.master)
    tokens, targets = synthetic_batch(cfg, 2, 128, seed=3)
    loss, saved = model.forward(tokens, targets)
    model.backward(saved)
    torch.cuda.synchronize()
    ref_loss, ref_grads = _torch_reference(model, tokens, targets)
    print(f"  loss {loss.item():.5f} ref {ref_loss:.5f}", flush=True)
    assert abs(loss.item() - ref_loss) <= 1e-2 * abs(ref_loss)
    worst = 0.0
    for name in model.offsets:
        got = model.embed_grad if name == "embed" else model.gr(name)
        e = rel_l2(got, ref_grads[name].cpu().numpy())
        worst = max(worst, e)
        print(f"  {name:12s} rel-L2 {e:.2e}", flush=True)
        assert e <= 6e-2, name
    print(f"  worst {worst:.2e}", flush=True)


def test_fused_projection_io_matches_copied_io():
    # 8 heads: the fused q/k/v/beta row (3 * 512 + 8 bf16) is whole 16-byte
    # pieces, so the EFLA calls read q, k, v and write their gradients in place
    # in it; with the copies they take packed tensors.  Same results, bit for bit.
    from ceo_amd.lm_step import EflaLM, LMConfig, synthetic_batch

    announce("lm step: fused-row EFLA io vs packed copies (8 heads)")
    cfg = LMConfig(vocab=256, d_model=128, n_layers=2, n_heads=8, head_dim=64, mlp=512)
    model = EflaLM(cfg, seed=5)
    model.master.mul_(4.0)
    model.weights.copy_(model.master)
    tokens, targets = synthetic_batch(cfg, 2, 160, seed=6)
    assert model.fused_io
    res = []
    for fused in (True, False):
        model.fused_io = fused
        loss, saved = model.forward(tokens, targets)
        model.backward(saved)
        torch.cuda.synchronize()
        res.append((loss.clone(), model.grads.clone(), model.embed_grad.clone()))
    assert torch.equal(res[0][0], res[1][0])
    assert torch.equal(res[0][1], res[1][1])
    assert torch.equal(res[0][2], res[1][2])
    assert torch.isfinite(res[0][1].float()).all()


def test_training_reduces_loss():
    from ceo_amd.lm_step import EflaLM, synthetic_batch

    announce("lm step: 8 AdamW steps on one batch")
    cfg = _small()
    cfg.lr = 3e-3
    model = EflaLM(cfg, seed=2)
    tokens, targets = synthetic_batch(cfg, 2, 128, seed=4)
    losses = [model.train_step(tokens, targets).item() for _ in range(8)]
    print("  losses", [f"{x:.3f}" for x in losses], flush=True)
    assert all(math.isfinite(x) for x in losses)
    assert abs(losses[0] - math.log(cfg.vocab)) < 0.5  # near-uniform predictions at init
    assert losses[-1] < losses[0] - 0.5
    # the bf16 copy the GEMMs read is the rounded fp32 master
    assert torch.equal(model.weights, model.master.to(torch.bfloat16))


def test_eval_forward_keeps_logits():
    """forward(train=False) returns the training forward's loss, keeps the
    logits (the fused cross-entropy would write dL/dlogits over them) and
    stores no activations."""
    from ceo_amd.lm_step import EflaLM, synthetic_batch

    announce("lm step: evaluation forward")
    cfg = _small()
    model = EflaLM(cfg, seed=7)
    tokens, targets = synthetic_batch(cfg, 2, 128, seed=8)
    loss_t, saved_t = model.forward(tokens, targets)
    loss_e, saved_e = model.forward(tokens, targets, train=False)
    torch.cuda.synchronize()
    print(f"  train-forward loss {loss_t.item():.6f} eval {loss_e.item():.6f}", flush=True)
    assert abs(loss_t.item() - loss_e.item()) <= 1e-5 * abs(loss_t.item())
    assert saved_e["layers"] == [] and "dlogits" not in saved_e
    logits = saved_e["logits"]
    assert logits.shape == (2 * 128, cfg.vocab) and torch.isfinite(logits.float()).all()
    # the kept logits are the logits: their softmax cross-entropy is the loss
    ref = torch.nn.functional.cross_entropy(logits.float(), targets.reshape(-1).long())
    assert abs(ref.item() - loss_e.item()) <= 1e-3 * abs(ref.item())
    # the training forward's rows hold dL/dlogits instead: each sums to ~0
    assert saved_t["dlogits"].float().sum(-1).abs().max().item() < 1e-2


def test_overlapped_update_matches_single_launch():
    """train_step's group-by-group AdamW on the update stream (beside the
    backward) leaves master weights, moments and the bf16 copy bit-identical
    to backward() followed by the single-launch update()."""
    from ceo_amd.lm_step import EflaLM, synthetic_batch

    announce("lm step: overlapped AdamW groups vs one launch")
    cfg = _small()
    cfg.lr = 3e-3
    tokens, targets = synthetic_batch(cfg, 2, 128, seed=11)
    runs = []
    for overlap in (True, False):
        model = EflaLM(cfg, seed=9)
        for _ in range(3):
            if overlap:
                model.train_step(tokens, targets)
            else:
                _, saved = model.forward(tokens, targets)
                model.backward(saved)
                model.update()
        torch.cuda.synchronize()
        runs.append((model.master, model.exp_avg, model.exp_avg_sq, model.weights))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    assert not torch.equal(runs[0][0], EflaLM(cfg, seed=9).master)  # the steps did update
