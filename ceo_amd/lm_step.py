"""Config-4 training step: a decoder LM with EFLA token mixing, run entirely on
this library's kernels.

Mirrors the reference's step structure -- ``Trainer.run`` calls
``forwardStep`` / ``backwardStep`` / ``updateStep`` per batch
(src/runtime/trainer.zig:152-185) -- over the model of
src/model/model.zig:152-204 (pre-LayerNorm block: LN -> EFLA -> residual ->
LN -> MLP up -> GELU -> MLP down -> residual) and ``EflaModel``
(model.zig:259-441: embedding, blocks, final LayerNorm, LM head).  Two
departures, both from the config the benchmark names: EFLA reads a query and a
per-token beta (Mode Q: q, k, v and beta projections, beta = sigmoid), and the
PRISM mixer the reference inserts after EFLA (model.zig:172) is not part of
the config and is left out.

Kernels: embedding (lm.hip), LayerNorm (layernorm.hip), GEMMs (gemm.hip, the
MLP's GELU and its derivative fused into the products' epilogues),
chunked EFLA with the forward's T, b and chunk states handed to the backward
(efla_q.hip, reading q, k, v and writing their gradients in place in the
fused q/k/v/beta projection rows), AdamW and the beta gate (elementwise.hip),
cross-entropy (lm.hip).  torch provides memory and views.

Parameters live in flat buffers: fp32 master weights, fp32 AdamW moments, a
bf16 copy that the GEMMs read (each weight a contiguous view into it) and a
bf16 gradient buffer the backward writes into.  ``update`` is one
``adamw_step_master`` launch over every parameter; ``train_step`` instead
updates each contiguous group of parameters (the LM head and final LayerNorm,
each block, the embedding) on a second stream as soon as the backward has
written its gradients, so the memory-bound optimizer runs beside the rest of
the backward.  AdamW is elementwise: the results are bit-identical.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import efla, nn


@dataclass
class LMConfig:
    vocab: int = 32000
    d_model: int = 1024
    n_layers: int = 24
    n_heads: int = 16
    head_dim: int = 64
    mlp: int = 4096
    ln_eps: float = 1e-5
    label_smoothing: float = 0.0
    lr: float = 3e-4
    weight_decay: float = 0.1
    beta1: float = 0.9
    beta2: float = 0.999
    adam_eps: float = 1e-8


_ALIGN = 64  # elements: every parameter view starts 256-byte aligned in fp32


class EflaLM:
    """Parameters, optimizer state and one explicit forward / backward / update."""

    def __init__(self, cfg: LMConfig, device="cuda", seed: int = 0):
        self.cfg = cfg
        self.device = torch.device(device)
        D, H, dh, F, V = cfg.d_model, cfg.n_heads, cfg.head_dim, cfg.mlp, cfg.vocab
        HD = H * dh
        self.proj = 3 * HD + H  # fused q, k, v, beta projection width
        # the EFLA kernels read q, k, v and write their gradients in place in
        # the fused rows when a row is whole 16-byte pieces
        self.fused_io = self.proj % 8 == 0
        specs = [("embed", (V, D), "normal", math.sqrt(1.0 / D))]
        for i in range(cfg.n_layers):
            specs += [
                (f"l{i}.ln1.w", (D,), "one", 0), (f"l{i}.ln1.b", (D,), "zero", 0),
                (f"l{i}.w_in", (D, self.proj), "normal", 0.02),
                (f"l{i}.w_o", (HD, D), "normal", 0.02 / math.sqrt(2 * cfg.n_layers)),
                (f"l{i}.ln2.w", (D,), "one", 0), (f"l{i}.ln2.b", (D,), "zero", 0),
                (f"l{i}.w_up", (D, F), "normal", 0.02), (f"l{i}.b_up", (F,), "zero", 0),
                (f"l{i}.w_down", (F, D), "normal", 0.02 / math.sqrt(2 * cfg.n_layers)),
                (f"l{i}.b_down", (D,), "zero", 0),
            ]
        specs += [("lnf.w", (D,), "one", 0), ("lnf.b", (D,), "zero", 0),
                  ("head", (D, V), "normal", 0.02)]
        self.offsets, off = {}, 0
        for name, shape, _, _ in specs:
            n = math.prod(shape)
            self.offsets[name] = (off, shape)
            off += (n + _ALIGN - 1) // _ALIGN * _ALIGN
        self.numel = off
        dev = self.device
        self.master = torch.zeros(off, dtype=torch.float32, device=dev)
        self.exp_avg = torch.zeros(off, dtype=torch.float32, device=dev)
        self.exp_avg_sq = torch.zeros(off, dtype=torch.float32, device=dev)
        self.weights = torch.zeros(off, dtype=torch.bfloat16, device=dev)
        self.grads = torch.zeros(off, dtype=torch.bfloat16, device=dev)
        g = torch.Generator(device=dev).manual_seed(seed)
        for name, shape, kind, std in specs:
            p = self._view(self.master, name)
            if kind == "normal":
                p.normal_(0.0, std, generator=g)
            elif kind == "one":
                p.fill_(1.0)
        self.weights.copy_(self.master)
        self.n_params = sum(math.prod(s) for _, s, _, _ in specs)
        self.step_count = 0
        self.embed_grad = torch.zeros(V, D, dtype=torch.float32, device=dev)
        self._ws = None
        self._ws_key = None
        # contiguous parameter groups in the order the backward completes them
        first = [self.offsets[f"l{i}.ln1.w"][0] for i in range(cfg.n_layers)]
        first.append(self.offsets["lnf.w"][0])
        self._groups = {"tail": (first[-1], off), "embed": (0, first[0])}
        for i in range(cfg.n_layers):
            self._groups[i] = (first[i], first[i + 1])
        self._upd_stream = None

    # -- parameter views ------------------------------------------------------
    def _view(self, buf: torch.Tensor, name: str) -> torch.Tensor:
        off, shape = self.offsets[name]
        return buf[off:off + math.prod(shape)].view(shape)

    def w(self, name):
        return self._view(self.weights, name)

    def gr(self, name):
        return self._view(self.grads, name)

    def _io(self, cols: torch.Tensor) -> torch.Tensor:
        """A column slice of a fused row as the EFLA kernels take it: itself
        when the rows are whole 16-byte pieces, else a packed copy."""
        return cols if self.fused_io else cols.contiguous()

    def _workspaces(self, B, T):
        """One backward-sized EFLA workspace per layer (T, b and chunk states
        handed from each layer's forward to its backward)."""
        if self._ws_key != (B, T):
            cfg = self.cfg
            q = torch.empty(B, T, cfg.n_heads, cfg.head_dim, dtype=torch.bfloat16,
                            device=self.device)
            self._ws = [efla.new_workspace(q, q) for _ in range(cfg.n_layers)]
            self._ws_key = (B, T)
        return self._ws

    # -- forward --------------------------------------------------------------
    def forward(self, tokens: torch.Tensor, targets: torch.Tensor, train: bool = True):
        """tokens, targets: (B, T) int32.  Returns (mean loss tensor, saved).

        With ``train`` (the step's forward) the cross-entropy also writes
        dL/dlogits over the logits in place, and ``saved`` holds what
        backward() needs.  With ``train=False`` (evaluation) the logits are
        kept (``saved["logits"]``) and no activation or gradient is stored."""
        cfg = self.cfg
        B, T = tokens.shape
        N, D, H, dh = B * T, cfg.d_model, cfg.n_heads, cfg.head_dim
        HD = H * dh
        ws = self._workspaces(B, T)
        x = nn.embedding_forward(tokens.reshape(-1), self.w("embed"))
        saved = {"tokens": tokens, "layers": []}
        for i in range(cfg.n_layers):
            L = f"l{i}."
            a, m1, r1 = nn.layernorm_forward(x, self.w(L + "ln1.w"), self.w(L + "ln1.b"),
                                             cfg.ln_eps, save_stats=True)
            p = nn.gemm_forward(a, self.w(L + "w_in"))
            # q, k, v are read in place from the fused projection's rows
            # (copied out when the row width is not whole 16-byte pieces)
            q, k, v = (self._io(p[:, j * HD:(j + 1) * HD]).view(B, T, H, dh) for j in range(3))
            beta = nn.sigmoid_gate_forward(p[:, 3 * HD:]).view(B, T, H)
            o, _ = efla.chunk_efla_fwd(q, k, v, beta, workspace=ws[i], save_states=train)
            o2 = o.view(N, HD)
            # x1 = x + o w_o with the residual added by the product's epilogue
            x1 = nn.gemm_ex(o2, self.w(L + "w_o"), torch.empty_like(x), c=x, beta=1.0)
            a2, m2, r2 = nn.layernorm_forward(x1, self.w(L + "ln2.w"), self.w(L + "ln2.b"),
                                              cfg.ln_eps, save_stats=True)
            # u = a2 w_up + b_up and gl = GELU(u) from one product (GELU in its epilogue)
            u, gl = nn.gemm_gelu_forward(a2, self.w(L + "w_up"), self.w(L + "b_up"))
            x2 = nn.gemm_ex(gl, self.w(L + "w_down"), torch.empty_like(x),
                            bias=self.w(L + "b_down"), c=x1, beta=1.0)
            if train:
                saved["layers"].append(dict(x=x, a=a, m1=m1, r1=r1, q=q, k=k, v=v, beta=beta,
                                            o=o2, x1=x1, a2=a2, m2=m2, r2=r2, u=u, g=gl))
            x = x2
        af, mf, rf = nn.layernorm_forward(x, self.w("lnf.w"), self.w("lnf.b"), cfg.ln_eps,
                                          save_stats=True)
        logits = nn.gemm_forward(af, self.w("head"))
        tflat = targets.reshape(-1)
        if not train:
            loss_rows = nn.cross_entropy_forward(logits, tflat, cfg.label_smoothing)
            saved.update(logits=logits)
            return loss_rows.sum(), saved
        # the loss and dL/dlogits of the summed rows from one read of the
        # logits, the gradient written over them (the backward needs no logits)
        loss_rows, dlogits = nn.cross_entropy_forward_backward(logits, tflat,
                                                               cfg.label_smoothing,
                                                               in_place=True)
        saved.update(x=x, af=af, mf=mf, rf=rf, dlogits=dlogits, targets=tflat)
        return loss_rows.sum(), saved

    # -- backward -------------------------------------------------------------
    def _update_group(self, key) -> None:
        """AdamW over one contiguous parameter group on the update stream, after
        everything the current stream has queued so far (its gradients)."""
        cfg = self.cfg
        lo, hi = self._groups[key]
        cur = torch.cuda.current_stream(self.device)
        self._upd_stream.wait_stream(cur)
        with torch.cuda.stream(self._upd_stream):
            nn.adamw_step_master(self.master[lo:hi], self.grads[lo:hi], self.exp_avg[lo:hi],
                                 self.exp_avg_sq[lo:hi], cfg.lr, cfg.beta1, cfg.beta2,
                                 cfg.adam_eps, cfg.weight_decay, self.step_count,
                                 param_bf16=self.weights[lo:hi])

    def backward(self, saved, update: bool = False) -> None:
        """Gradients of the mean loss into self.grads (bf16) / self.embed_grad;
        with ``update`` also the AdamW step, group by group on the update stream
        (the caller makes its stream wait for that one before reading the
        weights again, as ``train_step`` does)."""
        cfg = self.cfg
        if update:
            if self._upd_stream is None:
                self._upd_stream = torch.cuda.Stream(self.device)
            self.step_count += 1
        upd = self._update_group if update else (lambda key: None)
        B, T = saved["tokens"].shape
        N, D, H, dh = B * T, cfg.d_model, cfg.n_heads, cfg.head_dim
        HD = H * dh
        ws = self._workspaces(B, T)
        dlogits = saved["dlogits"]
        saved["dlogits"] = None
        daf, _, _ = nn.gemm_backward(dlogits, saved["af"], self.w("head"),
                                     out_b=self.gr("head"))
        del dlogits
        # b_down's gradient is the column sum of the layer output's gradient, so each
        # LayerNorm backward that produces that gradient also sums its columns
        top = cfg.n_layers - 1
        # parameter gradients straight into the bf16 gradient buffer
        dx, _, _ = nn.layernorm_backward(
            daf, saved["x"], self.w("lnf.w"), saved["mf"], saved["rf"],
            out_dx_colsum=self.gr(f"l{top}.b_down") if top >= 0 else None,
            out_dw=self.gr("lnf.w"), out_db=self.gr("lnf.b"))
        upd("tail")  # the LM head and final LayerNorm are read no more
        for i in reversed(range(cfg.n_layers)):
            L = f"l{i}."
            s = saved["layers"][i]
            # x2 = x1 + down(gelu(up(ln2(x1))))
            # du = (dx w_down^T) * GELU'(u) from one product (derivative in its epilogue)
            # and b_up's gradient (du's column sums) comes from the same epilogue
            du, _, _ = nn.gemm_gelu_backward(dx, s["g"], self.w(L + "w_down"), s["u"],
                                             out_b=self.gr(L + "w_down"),
                                             out_pre_bias=self.gr(L + "b_up"))
            da2, _, _ = nn.gemm_backward(du, s["a2"], self.w(L + "w_up"),
                                         out_b=self.gr(L + "w_up"))
            # dx1 = LN2's input gradient + the residual's dx, in one pass
            dx1, _, _ = nn.layernorm_backward(da2, s["x1"], self.w(L + "ln2.w"), s["m2"],
                                              s["r2"], residual=dx, out_dw=self.gr(L + "ln2.w"),
                                              out_db=self.gr(L + "ln2.b"))
            # x1 = x + o w_o, o = EFLA(q, k, v, beta)
            do, _, _ = nn.gemm_backward(dx1, s["o"], self.w(L + "w_o"), out_b=self.gr(L + "w_o"))
            # dq, dk, dv are written in place into the fused projection's gradient
            dp = torch.empty(N, 3 * HD + H, dtype=torch.bfloat16, device=self.device)
            views = tuple(self._io(dp[:, j * HD:(j + 1) * HD]).view(B, T, H, dh)
                          for j in range(3))
            _, _, _, dbeta, _ = efla.chunk_efla_bwd(
                s["q"], s["k"], s["v"], s["beta"], do.view(B, T, H, dh), workspace=ws[i],
                reuse_forward=True, reuse_states=True, grads_out=views)
            if not self.fused_io:
                for j in range(3):
                    dp[:, j * HD:(j + 1) * HD] = views[j].view(N, HD)
            nn.sigmoid_gate_backward(dbeta.view(N, H), s["beta"].view(N, H), dp[:, 3 * HD:])
            da, _, _ = nn.gemm_backward(dp, s["a"], self.w(L + "w_in"), out_b=self.gr(L + "w_in"))
            # dx = dx1 + LN1's input gradient
            dx, _, _ = nn.layernorm_backward(
                da, s["x"], self.w(L + "ln1.w"), s["m1"], s["r1"], residual=dx1,
                out_dx_colsum=self.gr(f"l{i - 1}.b_down") if i > 0 else None,
                out_dw=self.gr(L + "ln1.w"), out_db=self.gr(L + "ln1.b"))
            saved["layers"][i] = None
            upd(i)  # block i's gradients are complete (b_down's came from block i + 1)
        self.embed_grad.zero_()
        nn.embedding_backward(dx, saved["tokens"].reshape(-1), self.embed_grad)
        self.gr("embed").copy_(self.embed_grad)
        upd("embed")

    # -- update ---------------------------------------------------------------
    def update(self) -> None:
        """One AdamW step over every parameter (fp32 master, bf16 copy refreshed)."""
        cfg = self.cfg
        self.step_count += 1
        nn.adamw_step_master(self.master, self.grads, self.exp_avg, self.exp_avg_sq, cfg.lr,
                             cfg.beta1, cfg.beta2, cfg.adam_eps, cfg.weight_decay,
                             self.step_count, param_bf16=self.weights)

    def train_step(self, tokens: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
        """forwardStep, backwardStep, updateStep; returns the loss (device scalar).
        The update runs group by group beside the backward (see ``backward``)."""
        loss, saved = self.forward(tokens, targets)
        self.backward(saved, update=True)
        torch.cuda.current_stream(self.device).wait_stream(self._upd_stream)
        return loss


def synthetic_batch(cfg: LMConfig, batch: int, seq: int, seed: int, device="cuda"):
    """Token ids uniform over the vocabulary; targets are the next token."""
    g = torch.Generator(device=device).manual_seed(seed)
    ids = torch.randint(0, cfg.vocab, (batch, seq + 1), generator=g, device=device,
                        dtype=torch.int32)
    return ids[:, :-1].contiguous(), ids[:, 1:].contiguous()


def step_flops(cfg: LMConfig, tokens: int, seq: int) -> float:
    """Model FLOPs of one training step: 6 x (GEMM weights) per token, plus
    EFLA at 3 F_fwd per (token, head) with F_fwd = C(6K + 4V) + 6KV + 2C^2/3."""
    D, H, dh, F, V = cfg.d_model, cfg.n_heads, cfg.head_dim, cfg.mlp, cfg.vocab
    gemm_w = cfg.n_layers * (D * (3 * H * dh + H) + H * dh * D + 2 * D * F) + D * V
    C = 64
    f_efla = C * (6 * dh + 4 * dh) + 6 * dh * dh + 2 * C * C / 3
    return 6.0 * gemm_w * tokens + 3.0 * f_efla * tokens * H * cfg.n_layers
