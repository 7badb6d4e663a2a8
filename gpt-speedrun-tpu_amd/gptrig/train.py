"""The GPT training step on one MI355X, composed from the gfx950 kernels.

Restates ``recipes/reference/train.py``: ``init_params`` (``:865-901``),
``gpt_hidden`` (``:1096-1176``), ``cross_entropy`` with the tiled loss
(``:1194-1210``) and ``_apply_training_update`` (``:1362-1457``).

Memory layout (HBM):
* one float32 arena holds every parameter, each tensor starting on a
  4096-element chunk boundary, plus same-shaped float32 arenas for the
  gradient and the two Adam moments;
* a bfloat16 shadow arena holds ``bf16(param)``, refreshed by the AdamW kernel,
  which is exactly the reference's ``W.astype(bfloat16)`` at use;
* activations are ``[tokens, features]`` bf16 row-major; attention reads
  q/k/v in place from the ``[tokens, 3*d_model]`` projection (BHSD strides)
  and writes its output as ``[tokens, d_model]``.

The forward and backward passes are explicit (no autograd tape): RMSNorm,
RoPE, attention, GELU, the LM-head cross-entropy, the embedding scatter and
AdamW are HIP kernels; the forward and input-gradient projections are
hipBLASLt GEMMs through torch, the weight gradients the HIP GEMM with
split-K float32 accumulation into the gradient arena.  Weight gradients accumulate in float32 across micro-batches; the
global batch is split into equal micro-batches whose mean losses are averaged,
which equals the reference's single-batch token mean.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .attention import attention_softmax_scale, document_segments
from .kernels import linear_cross_entropy as lce
from .nn import add_rmsnorm_forward, normal, rmsnorm_backward, rmsnorm_forward, rope_tables
from .optim import OptimizerConfig, effective_adam_betas, learning_rate, tensor_hparams

BF16 = torch.bfloat16
F32 = torch.float32
CHUNK = 4096
BLOCK_LEAVES = ("ln1_scale", "qkv_w", "qkv_b", "attn_w", "attn_b",
                "ln2_scale", "mlp_up_w", "mlp_up_b", "mlp_down_w", "mlp_down_b")
DENSE_LINEARS = ("qkv_w", "attn_w", "mlp_up_w", "mlp_down_w")


@dataclass(frozen=True)
class GPTConfig:
    """Model/optimizer fields of the reference ``Config`` (``train.py:176-282``)."""

    layers: int = 12
    heads: int = 12
    d_model: int = 768
    mlp_mult: int = 4
    vocab_size: int = 50304
    semantic_vocab_size: int = 50304
    seq_len: int = 1024
    batch_size: int = 128
    micro_batch_size: int = 32
    parameterization: str = "standard"
    base_width: int = 768
    base_depth: int = 12
    depth_alpha: float = 0.0
    init_std: float = 0.02
    attention_scale: str = "inverse_sqrt_head_dim"
    embeddings: str = "untied"
    vocab_tile_size: int = 2048
    document_masking: bool = False
    document_boundary_token: int = 50256
    # Routed (MoE) MLPs, recipes/reference_moe/train.py:242-245: 0 = dense.
    experts: int = 0
    expert_top_k: int = 2
    expert_mult: int = 2
    router_aux_coefficient: float = 0.01
    # FLCE working set.  False (the default): bounded like the reference's
    # tiled loss (linear_cross_entropy.py:1-24, at most [tokens, vocab_tile_size]
    # fp32 logits live): the micro-batch's tokens are cut into chunks whose
    # kept fp16 probabilities [vocab, chunk] take at most tokens x
    # vocab_tile_size x 4 bytes, and each chunk's forward and backward run
    # back to back (the loss is the step's last node, so its cotangent is
    # known).  True: one chunk over all tokens ([vocab, tokens] fp16, 6.6 GB
    # at 65536 tokens; fastest on one MI355X).
    flce_whole_vocab: bool = False
    optimizer: OptimizerConfig = field(default_factory=OptimizerConfig)

    @property
    def head_dim(self) -> int:
        return self.d_model // self.heads

    @property
    def width_multiplier(self) -> float:
        return self.d_model / float(self.base_width)

    @property
    def depth_multiplier(self) -> float:
        return self.layers / float(self.base_depth)

    def validate(self) -> None:
        if self.d_model % self.heads:
            raise ValueError("d_model must be divisible by heads")
        if self.head_dim % 2:
            raise ValueError("head dimension must be even for RoPE")
        if self.semantic_vocab_size > self.vocab_size:
            raise ValueError("semantic_vocab_size must not exceed vocab_size")
        if self.batch_size % self.micro_batch_size:
            raise ValueError("micro_batch_size must divide batch_size")
        if self.head_dim not in (64, 128) or self.d_model % 64:
            raise ValueError("the HIP step needs head_dim in {64, 128} and d_model % 64 == 0")
        if self.experts:
            # reference_moe/train.py:362-371
            if self.expert_top_k > self.experts:
                raise ValueError("expert_top_k must not exceed experts")
            if self.expert_top_k * self.expert_mult != self.mlp_mult:
                raise ValueError("must satisfy expert_top_k * expert_mult == mlp_mult so active MLP FLOPs match "
                                 "the dense tier")
            if self.experts > 16 or self.expert_top_k > 8 or self.d_model * self.experts > 8192:
                raise ValueError("the HIP router needs experts <= 16, expert_top_k <= 8, d_model * experts <= 8192")
            if self.micro_batch_size != self.batch_size:
                # The balance loss is a product of two global-batch means
                # (reference_moe/train.py:1292-1296); one pass keeps it exact.
                raise ValueError("a routed model takes the whole batch in one pass: micro_batch_size must equal "
                                 "batch_size")


def init_params(config: GPTConfig, seed: int) -> dict[str, np.ndarray]:
    """``init_params`` (``train.py:865-901``) as a flat ``{path: float32}``
    mapping in the reference's draw order (numpy PCG64, so bit-identical)."""

    rng = np.random.default_rng(seed)
    d = config.d_model
    hidden = config.mlp_mult * d
    hidden_scale = (config.init_std / math.sqrt(config.width_multiplier)
                    if config.parameterization == "completep_fixed_tpp_v1" else 0.02)
    flat: dict[str, np.ndarray] = {}
    blocks = []
    for _ in range(config.layers):
        block = {
            "ln1_scale": np.ones((d,), np.float32),
            "qkv_w": normal(rng, (d, 3 * d), hidden_scale),
            "qkv_b": np.zeros((3 * d,), np.float32),
            "attn_w": normal(rng, (d, d), hidden_scale),
            "attn_b": np.zeros((d,), np.float32),
            "ln2_scale": np.ones((d,), np.float32),
        }
        if config.experts:
            # reference_moe/train.py:894-944: the router, then the stacked experts.
            E, eh = config.experts, config.expert_mult * d
            block["router_w"] = normal(rng, (d, E), hidden_scale)
            block["expert_up_w"] = normal(rng, (E, d, eh), hidden_scale)
            block["expert_up_b"] = np.zeros((E, eh), np.float32)
            block["expert_down_w"] = normal(rng, (E, eh, d), hidden_scale)
            block["expert_down_b"] = np.zeros((E, d), np.float32)
        else:
            block["mlp_up_w"] = normal(rng, (d, hidden), hidden_scale)
            block["mlp_up_b"] = np.zeros((hidden,), np.float32)
            block["mlp_down_w"] = normal(rng, (hidden, d), hidden_scale)
            block["mlp_down_b"] = np.zeros((d,), np.float32)
        blocks.append(block)
    flat["token_embedding"] = normal(rng, (config.vocab_size, d), config.init_std)
    for i, block in enumerate(blocks):
        for name, value in block.items():
            flat[f"blocks/{i}/{name}"] = value
    flat["final_ln_scale"] = np.ones((d,), np.float32)
    if config.embeddings == "untied":
        flat["output_embedding"] = normal(rng, (config.vocab_size, d), config.init_std / config.width_multiplier)
    return flat


def flce_token_chunk(tokens: int, vocab: int, vocab_tile_size: int, whole: bool) -> int:
    """Tokens per kept-softmax FLCE chunk of a micro-batch.

    ``whole``: all of them.  Otherwise the largest multiple of 64 tokens whose
    kept buffer (``gptrig_flce_keep_bytes``: fp16 probabilities over the
    padded vocabulary plus the per-row maxima) fits ``tokens x
    vocab_tile_size x 4`` bytes, the reference's fp32 ``[tokens,
    vocab_tile_size]`` live logits (``linear_cross_entropy.py:1-24``), at
    least 64; then evened out over the chunks it needs.
    """

    if whole:
        return tokens
    per64 = _lib.query("gptrig_flce_keep_bytes", 64, vocab)
    budget = tokens * vocab_tile_size * 4
    cap = max(1, budget // per64) * 64
    if cap >= tokens:
        return tokens
    share = -(-tokens // -(-tokens // cap))  # an even share of the chunks needed, <= cap
    return -(-share // 64) * 64  # still <= cap, a multiple of 64


class ParamArena:
    """Flat float32 parameter / gradient / moment arenas and the bf16 shadow."""

    def __init__(self, flat: dict[str, np.ndarray], device):
        self.paths = list(flat)
        self.shapes = {k: tuple(v.shape) for k, v in flat.items()}
        self.offsets: dict[str, int] = {}
        off = 0
        for k, v in flat.items():
            self.offsets[k] = off
            off += (v.size + CHUNK - 1) // CHUNK * CHUNK
        self.total = off
        self.n_chunks = off // CHUNK
        host = torch.zeros(off, dtype=F32)
        chunk_tensor = np.zeros(self.n_chunks, np.int32)
        for i, (k, v) in enumerate(flat.items()):
            o = self.offsets[k]
            host[o:o + v.size] = torch.from_numpy(np.ascontiguousarray(v).reshape(-1))
            chunk_tensor[o // CHUNK:(o + v.size + CHUNK - 1) // CHUNK] = i
        self.p = host.to(device)
        self.g = torch.zeros(off, dtype=F32, device=device)
        self.m = torch.zeros(off, dtype=F32, device=device)
        self.v = torch.zeros(off, dtype=F32, device=device)
        self.shadow = torch.empty(off, dtype=BF16, device=device)
        _lib.call("gptrig_cast_f32_bf16", self.p.data_ptr(), self.shadow.data_ptr(), off, _lib.stream())
        self.chunk_tensor = torch.from_numpy(chunk_tensor).to(device)
        # [d_out, d_in] copies of the block linear weights: hipBLASLt runs the
        # forward x W as x (W^T)^T 10-20% faster from this layout, while dX = dy W^T
        # is fastest from the original one, so both are kept.
        self.transposed = {k: torch.empty((s[1], s[0]), dtype=BF16, device=device)
                           for k, s in self.shapes.items()
                           if k.startswith("blocks/") and k.rsplit("/", 1)[-1] in DENSE_LINEARS}
        self.refresh_transposed()

    def refresh_transposed(self) -> None:
        for k, t in self.transposed.items():
            rows, cols = self.shapes[k]
            _lib.call("gptrig_transpose_bf16", self.w(k).data_ptr(), t.data_ptr(), rows, cols, _lib.stream())

    def wt(self, path):
        """bf16 ``param.T`` of a block linear weight, refreshed after every update."""
        return self.transposed[path]

    def _view(self, arena: torch.Tensor, path: str) -> torch.Tensor:
        o = self.offsets[path]
        shape = self.shapes[path]
        return arena[o:o + int(np.prod(shape))].view(shape)

    def param(self, path):
        return self._view(self.p, path)

    def grad(self, path):
        return self._view(self.g, path)

    def w(self, path):
        """bf16 shadow (``param.astype(bfloat16)``)."""
        return self._view(self.shadow, path)

    def numel(self) -> int:
        return sum(int(np.prod(s)) for s in self.shapes.values())


class GPTTrainer:
    """One-GPU training step for the reference GPT (``train_step``, ``train.py:1460-1472``)."""

    def __init__(self, config: GPTConfig, seed: int = 0, device: str = "cuda:0", history_steps: int | None = None):
        config.validate()
        self.config = config
        self.device = torch.device(device)
        self.arena = ParamArena(init_params(config, seed), self.device)
        self.step_count = 0
        self.beta1, self.beta2 = effective_adam_betas(config.optimizer)
        self.hparams = torch.from_numpy(
            tensor_hparams(self.arena.paths, config.optimizer, config.parameterization, config.width_multiplier,
                           config.depth_multiplier, config.depth_alpha)).to(self.device)
        steps = history_steps or config.optimizer.steps
        self.history = torch.zeros((steps, 3), dtype=F32, device=self.device)
        self.loss = torch.zeros(1, dtype=F32, device=self.device)
        self.sq_partials = torch.zeros(self.arena.n_chunks, dtype=F32, device=self.device)
        # Weight gradients are taken once per step over all micro-batches: each
        # micro-batch writes the inputs and output-gradients of the block
        # linears into its rows of these [batch*seq, width] buffers, and the
        # dW/db GEMMs then run with the whole global batch as their K
        # dimension (same sums as per-micro-batch accumulation, in a different
        # fp32 order; four times fewer, four times longer split-K launches).
        T = config.batch_size * config.seq_len
        d, f = config.d_model, config.mlp_mult * config.d_model
        widths = {"qkv": (d, 3 * d), "attn": (d, d)}
        if not config.experts:
            widths.update({"mlp_up": (d, f), "mlp_down": (f, d)})
        self.linears = tuple(widths)
        self.lin_in = [{k: torch.empty((T, a), dtype=BF16, device=self.device) for k, (a, _) in widths.items()}
                       for _ in range(config.layers)]
        self.lin_dout = [{k: torch.empty((T, b), dtype=BF16, device=self.device) for k, (_, b) in widths.items()}
                         for _ in range(config.layers)]
        self.norm = torch.zeros(1, dtype=F32, device=self.device)
        self.clip = torch.ones(1, dtype=F32, device=self.device)
        self.head_path = "output_embedding" if config.embeddings == "untied" else "token_embedding"
        self.scale = attention_softmax_scale(config.attention_scale, config.head_dim)
        self.residual_scale = config.depth_multiplier ** (-config.depth_alpha)
        self._ws: dict[str, torch.Tensor] = {}
        self.router_load = None  # [layers, experts] f32 of the last step (routed models)
        self.timers = None  # optional {name: list[(start_event, end_event)]}
        # A layer's weight gradients can run as soon as the last micro-batch's
        # backward has written that layer's output-gradients: they go to a
        # second stream (default priority, like every stream here) and overlap
        # the backward of the layers below, whose attention and elementwise
        # launches leave the matrix cores partly idle.  One event per layer
        # marks the point; the step's optimizer update waits for the stream.
        self.wgrad_stream = torch.cuda.Stream(device=self.device)
        self._layer_ready = [torch.cuda.Event() for _ in range(config.layers)]

    # -- helpers -----------------------------------------------------------------
    def _workspace(self, name: str, nbytes: int) -> torch.Tensor:
        ws = self._ws.get(name)
        if ws is None or ws.numel() < nbytes:
            ws = _lib.workspace(nbytes, self.device)
            self._ws[name] = ws
        return ws

    def _timed(self, name):
        timers = self.timers

        class _Ctx:
            def __enter__(self_inner):
                if timers is not None:
                    self_inner.s = torch.cuda.Event(enable_timing=True)
                    self_inner.e = torch.cuda.Event(enable_timing=True)
                    self_inner.s.record()

            def __exit__(self_inner, *exc):
                if timers is not None:
                    self_inner.e.record()
                    timers.setdefault(name, []).append((self_inner.s, self_inner.e))

        return _Ctx()

    # -- routed MLP (reference_moe/train.py:1230-1307) ---------------------------------
    def _routed_forward(self, p: str, xn2: torch.Tensor):
        """The routed MLP of block ``p`` on the normalised rows ``xn2`` [N, d]:
        fp32 router logits, top-k routing with the stable bucket sort, the two
        grouped expert GEMMs (bias + GELU, bias) and the gated combine.  Returns
        the bf16 [N, d] block output and what the backward and the balance loss
        need."""

        c, A = self.config, self.arena
        N, d = xn2.shape
        E, k, eh = c.experts, c.expert_top_k, c.expert_mult * c.d_model
        R = N * k
        dev, s = self.device, _lib.stream()
        logits = torch.empty((N, E), dtype=F32, device=dev)
        _lib.call("gptrig_moe_router_logits", xn2.data_ptr(), A.param(p + "router_w").data_ptr(), logits.data_ptr(),
                  N, d, E, s)
        probs = torch.empty((N, E), dtype=F32, device=dev)
        chosen = torch.empty((N, k), dtype=torch.int32, device=dev)
        gate = torch.empty((N, k), dtype=F32, device=dev)
        counts = torch.empty(E, dtype=torch.int32, device=dev)
        order = torch.empty(R, dtype=torch.int32, device=dev)
        rows = torch.empty(R, dtype=torch.int32, device=dev)
        position = torch.empty(R, dtype=torch.int32, device=dev)
        ws = self._workspace("moe_route", _lib.query("gptrig_moe_route_workspace_bytes", N, E, k))
        _lib.call("gptrig_moe_route", logits.data_ptr(), probs.data_ptr(), chosen.data_ptr(), gate.data_ptr(),
                  counts.data_ptr(), order.data_ptr(), rows.data_ptr(), position.data_ptr(), ws.data_ptr(), ws.numel(),
                  N, E, k, s)
        grouped = torch.empty((R, d), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_gather_rows", xn2.data_ptr(), rows.data_ptr(), grouped.data_ptr(), R, d, s)
        pre = torch.empty((R, eh), dtype=BF16, device=dev)
        hidden = torch.empty((R, eh), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_gmm", grouped.data_ptr(), d, A.w(p + "expert_up_w").data_ptr(), 0, counts.data_ptr(),
                  A.w(p + "expert_up_b").data_ptr(), 1, hidden.data_ptr(), pre.data_ptr(), eh, R, d, eh, E, s)
        out = torch.empty((R, d), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_gmm", hidden.data_ptr(), eh, A.w(p + "expert_down_w").data_ptr(), 0, counts.data_ptr(),
                  A.w(p + "expert_down_b").data_ptr(), 0, out.data_ptr(), None, d, R, eh, d, E, s)
        combined = torch.empty((N, d), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_combine", out.data_ptr(), position.data_ptr(), gate.data_ptr(), combined.data_ptr(), N,
                  d, k, s)
        mean_probability = torch.empty(E, dtype=F32, device=dev)
        load = torch.empty(E, dtype=F32, device=dev)
        summary = torch.empty(3, dtype=F32, device=dev)
        _lib.call("gptrig_moe_stats", logits.data_ptr(), probs.data_ptr(), gate.data_ptr(), counts.data_ptr(), N, E,
                  k, mean_probability.data_ptr(), load.data_ptr(), summary.data_ptr(), s)
        return combined, (probs, chosen, gate, counts, position, grouped, pre, hidden, out, mean_probability, load)

    def _routed_backward(self, p: str, xn2: torch.Tensor, state, dm: torch.Tensor) -> torch.Tensor:
        """VJP of the routed MLP of block ``p`` for the block-output gradient
        ``dm`` [N, d] plus the balance loss's share (coefficient / layers times
        E * load, the gradient of the mean probability; the load carries none).
        Expert and router gradients accumulate into the gradient arena; returns
        the bf16 gradient of ``xn2``."""

        c, A = self.config, self.arena
        probs, chosen, gate, counts, position, grouped, pre, hidden, out, _, load = state
        N, d = xn2.shape
        E, k, eh = c.experts, c.expert_top_k, c.expert_mult * c.d_model
        R = N * k
        dev, s = self.device, _lib.stream()
        dout = torch.empty((R, d), dtype=BF16, device=dev)
        dgate = torch.empty(R, dtype=F32, device=dev)
        _lib.call("gptrig_moe_combine_bwd", dm.data_ptr(), out.data_ptr(), position.data_ptr(), gate.data_ptr(),
                  dout.data_ptr(), dgate.data_ptr(), N, d, k, s)
        dpre = torch.empty((R, eh), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_gmm", dout.data_ptr(), d, A.w(p + "expert_down_w").data_ptr(), 1, counts.data_ptr(),
                  None, 2, dpre.data_ptr(), pre.data_ptr(), eh, R, d, eh, E, s)
        # The expert weight gradients go to the weight-gradient stream, like
        # the dense linears': they overlap the rest of this block's backward
        # and the blocks below.  Their inputs are per-call tensors, so each
        # is marked as in use by that stream (the allocator then reuses none
        # of them before the stream's kernels have run).
        main, side = torch.cuda.current_stream(dev), self.wgrad_stream
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ws = _lib.stream()
            _lib.call("gptrig_moe_gmm_dw", hidden.data_ptr(), eh, dout.data_ptr(), d, counts.data_ptr(),
                      A.grad(p + "expert_down_w").data_ptr(), A.grad(p + "expert_down_b").data_ptr(), R, eh, d, E,
                      ws)
            _lib.call("gptrig_moe_gmm_dw", grouped.data_ptr(), d, dpre.data_ptr(), eh, counts.data_ptr(),
                      A.grad(p + "expert_up_w").data_ptr(), A.grad(p + "expert_up_b").data_ptr(), R, d, eh, E, ws)
        for t in (hidden, dout, grouped, dpre, counts):
            t.record_stream(side)
        dgrouped = torch.empty((R, d), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_gmm", dpre.data_ptr(), eh, A.w(p + "expert_up_w").data_ptr(), 1, counts.data_ptr(),
                  None, 0, dgrouped.data_ptr(), None, d, R, eh, d, E, s)
        dxn2 = torch.empty((N, d), dtype=BF16, device=dev)
        _lib.call("gptrig_moe_gather_bwd", dgrouped.data_ptr(), position.data_ptr(), dxn2.data_ptr(), N, d, k, s)
        dmp = (load * (c.router_aux_coefficient * E / c.layers)).contiguous()
        _lib.call("gptrig_moe_router_bwd", xn2.data_ptr(), A.param(p + "router_w").data_ptr(), probs.data_ptr(),
                  chosen.data_ptr(), gate.data_ptr(), dgate.data_ptr(), dmp.data_ptr(), dxn2.data_ptr(),
                  A.grad(p + "router_w").data_ptr(), N, d, E, k, s)
        return dxn2

    # -- forward / backward of one micro-batch --------------------------------------
    def _forward(self, tokens: torch.Tensor, micro: int):
        """Blocks and final norm of one micro-batch (``gpt_hidden``, ``train.py:1096-1176``).

        Returns ``(tok, seg, x, xf, rstdf, saved)``: the flat int32 tokens, the
        document segments (or ``None``), the last residual stream, its final
        norm with the rstd, and each layer's saved activations.  The inputs of
        the block linears go to this micro-batch's rows of ``lin_in``.
        """

        c = self.config
        A = self.arena
        Bm, S = tokens.shape
        N, d, H, D = Bm * S, c.d_model, c.heads, c.head_dim
        rows = slice(micro * N, (micro + 1) * N)
        lin_in = [{k: t[rows] for k, t in layer.items()} for layer in self.lin_in]
        stream = _lib.stream()
        tok = tokens.reshape(-1).to(torch.int32).contiguous()
        seg = document_segments(tokens, c.document_boundary_token).contiguous() if c.document_masking else None

        x = torch.empty((N, d), dtype=BF16, device=self.device)
        _lib.call("gptrig_embedding_fwd", tok.data_ptr(), A.w("token_embedding").data_ptr(), x.data_ptr(), N, d,
                  c.vocab_size, stream)
        # strides (elements) of q/k/v inside the [N, 3d] projection, of o in [N, d]
        st_qkv = (S * 3 * d, D, 3 * d)
        st_o = (S * d, D, d)
        attn_strides = torch.tensor([*st_qkv, *st_qkv, *st_qkv, *st_o], dtype=torch.int64)
        saved = []
        # Each residual add runs fused with the norm after it (ln2 of the same
        # block, ln1 of the next, or the final norm).
        if c.layers == 0:
            xf, rstdf = rmsnorm_forward(x, A.w("final_ln_scale"))
        else:
            xn1, rstd1 = rmsnorm_forward(x, A.w("blocks/0/ln1_scale"), out=lin_in[0]["qkv"])
        # The QKV projection is this library's GEMM with the bias add and the
        # RoPE of q and k in its epilogue (gptrig_linear_rope: 281 against
        # 301 us at config D in isolation for hipBLASLt plus the bias + RoPE
        # pass; the same step time either way).  The other
        # linears are hipBLASLt GEMMs alone (bf16 output), their bias added,
        # with its own rounding as in rig/nn.py:55-56, by the pass that
        # consumes them (the GELU, the residual add).
        rope_c, rope_s = rope_tables(S, D, self.device)
        for i in range(c.layers):
            p = f"blocks/{i}/"
            qkv = torch.empty((N, 3 * d), dtype=BF16, device=self.device)
            _lib.call("gptrig_linear_rope", xn1.data_ptr(), d, A.wt(p + "qkv_w").data_ptr(), d, 1,
                      A.w(p + "qkv_b").data_ptr(), qkv.data_ptr(), 3 * d, N, d, 3 * d, rope_c.data_ptr(),
                      rope_s.data_ptr(), S, 2 * d, D, stream)
            o = lin_in[i]["attn"]
            lse = torch.empty((Bm, H, S), dtype=F32, device=self.device)
            with self._timed("attn_fwd"):
                _lib.call("gptrig_attn_fwd", qkv.data_ptr(), qkv[:, d:].data_ptr(), qkv[:, 2 * d:].data_ptr(),
                          _lib.ptr(seg), o.data_ptr(), lse.data_ptr(), Bm, H, S, D, attn_strides.data_ptr(),
                          self.scale, stream)
            x1, xn2, rstd2 = add_rmsnorm_forward(x, torch.mm(o, A.wt(p + "attn_w").t()),
                                                 self.residual_scale, A.w(p + "ln2_scale"),
                                                 out=None if c.experts else lin_in[i]["mlp_up"],
                                                 branch_bias=A.w(p + "attn_b"))
            if c.experts:
                down, mlp_state = self._routed_forward(p, xn2)
            else:
                h = torch.mm(xn2, A.wt(p + "mlp_up_w").t())  # the pre-activation before its bias
                g = lin_in[i]["mlp_down"]
                _lib.call("gptrig_bias_gelu_fwd", h.data_ptr(), A.w(p + "mlp_up_b").data_ptr(), g.data_ptr(),
                          h.shape[0], h.shape[1], stream)
                down = torch.mm(g, A.wt(p + "mlp_down_w").t())
                mlp_state = (h, g)
            down_b = None if c.experts else A.w(p + "mlp_down_b")
            if i + 1 < c.layers:
                x2, xn1_next, rstd1_next = add_rmsnorm_forward(x1, down, self.residual_scale,
                                                               A.w(f"blocks/{i + 1}/ln1_scale"),
                                                               out=lin_in[i + 1]["qkv"], branch_bias=down_b)
            else:
                x2, xf, rstdf = add_rmsnorm_forward(x1, down, self.residual_scale, A.w("final_ln_scale"),
                                                    branch_bias=down_b)
            saved.append((x, xn1, rstd1, qkv, o, lse, x1, xn2, rstd2, mlp_state))
            x = x2
            if i + 1 < c.layers:
                xn1, rstd1 = xn1_next, rstd1_next
        return tok, seg, x, xf, rstdf, saved

    def _forward_backward(self, tokens: torch.Tensor, targets: torch.Tensor, loss_weight: float, micro: int,
                          mark_layers: bool = False) -> None:
        c = self.config
        A = self.arena
        Bm, S = tokens.shape
        N, d, H, D = Bm * S, c.d_model, c.heads, c.head_dim
        rows = slice(micro * N, (micro + 1) * N)
        lin_dout = [{k: t[rows] for k, t in layer.items()} for layer in self.lin_dout]
        stream = _lib.stream()
        tgt = targets.reshape(-1).to(torch.int32).contiguous()
        if tgt.data_ptr() % 16:  # a row slice of a window: the FLCE backward reads 16-byte groups
            tgt = tgt.clone()
        tok, seg, x, xf, rstdf, saved = self._forward(tokens, micro)
        st_qkv = (S * 3 * d, D, 3 * d)
        st_o = (S * d, D, d)
        bwd_strides = torch.tensor([*st_qkv, *st_qkv, *st_qkv, *st_o, *st_o, *st_qkv, *st_qkv, *st_qkv],
                                   dtype=torch.int64)
        head = A.w(self.head_path)
        losses = torch.empty(N, dtype=F32, device=self.device)
        lse_ce = torch.empty(N, dtype=F32, device=self.device)
        dxf = torch.empty((N, d), dtype=BF16, device=self.device)
        # Kept softmax: the forward keeps its probabilities (fp16 [vocab,
        # chunk]) and the backward rescales them into the logit gradient
        # instead of recomputing the logits GEMM; each token chunk runs its
        # forward and backward back to back (bounded by vocab_tile_size unless
        # flce_whole_vocab).  The head gradient accumulates over chunks.
        chunk = flce_token_chunk(N, c.vocab_size, c.vocab_tile_size, c.flce_whole_vocab) \
            if d % 128 == 0 and N % 8 == 0 else 0
        if chunk:
            keep = self._workspace("flce_keep", _lib.query("gptrig_flce_keep_bytes", chunk, c.vocab_size))
            ws = self._workspace("flce_fwd", _lib.query("gptrig_flce_fwd_workspace_bytes", chunk, d, c.vocab_size))
            ws_b = self._workspace("flce_bwd_keep", _lib.query("gptrig_flce_bwd_keep_workspace_bytes", chunk, d))
            dw = A.grad(self.head_path)
            with self._timed("flce"):
                for c0 in range(0, N, chunk):
                    n = min(chunk, N - c0)
                    hp, tp = xf[c0:].data_ptr(), tgt[c0:].data_ptr()
                    _lib.call("gptrig_flce_fwd_keep", hp, head.data_ptr(), tp, losses[c0:].data_ptr(),
                              lse_ce[c0:].data_ptr(), keep.data_ptr(), keep.numel(), ws.data_ptr(), ws.numel(), n, d,
                              c.vocab_size, c.semantic_vocab_size, stream)
                    _lib.call("gptrig_flce_bwd_keep", hp, head.data_ptr(), tp, lse_ce[c0:].data_ptr(), None,
                              loss_weight, dxf[c0:].data_ptr(), dw.data_ptr(), 1, keep.data_ptr(), keep.numel(),
                              ws_b.data_ptr(), ws_b.numel(), n, d, c.vocab_size, c.semantic_vocab_size, stream)
        else:
            ws = self._workspace("flce_fwd", _lib.query("gptrig_flce_fwd_workspace_bytes", N, d, c.vocab_size))
            with self._timed("flce"):
                _lib.call("gptrig_flce_fwd", xf.data_ptr(), head.data_ptr(), tgt.data_ptr(), losses.data_ptr(),
                          lse_ce.data_ptr(), ws.data_ptr(), ws.numel(), N, d, c.vocab_size, c.semantic_vocab_size,
                          stream)
        _lib.call("gptrig_weighted_sum", losses.data_ptr(), N, loss_weight, self.loss.data_ptr(), stream)
        if c.experts:
            # The per-layer expert load of the step (the reference's router row,
            # reference_moe/train.py:1881-1908), kept on the device.
            self.router_load = torch.stack([st[-1] for *_, st in saved])
            if c.router_aux_coefficient:
                # + coefficient x mean over layers of E * sum(load * P) (:1347-1371, :1557-1558)
                aux = sum((st[-1] * st[-2]).sum() for *_, st in saved)
                self.loss.add_(aux * (c.router_aux_coefficient * c.experts / c.layers))

        # ---- backward ----
        if not chunk:
            # (d not a multiple of 128) the recompute backward over vocabulary
            # chunks of vocab_tile_size, or one chunk with flce_whole_vocab.
            vchunk = lce.grad_chunk(N, c.vocab_size) if c.flce_whole_vocab else lce.chunk_for(c.vocab_tile_size)
            ws = self._workspace("flce_bwd",
                                 _lib.query("gptrig_flce_bwd_workspace_bytes", N, d, c.vocab_size, vchunk))
            with self._timed("flce"):
                _lib.call("gptrig_flce_bwd", xf.data_ptr(), head.data_ptr(), tgt.data_ptr(), lse_ce.data_ptr(), None,
                          loss_weight, dxf.data_ptr(), A.grad(self.head_path).data_ptr(), 1, ws.data_ptr(),
                          ws.numel(), N, d, c.vocab_size, c.semantic_vocab_size, vchunk, stream)
        unit = self.residual_scale == 1.0
        top = lin_dout[c.layers - 1]["mlp_down"] if unit and not c.experts else None
        dx, _ = rmsnorm_backward(dxf, x, A.w("final_ln_scale"), rstdf, A.grad("final_ln_scale"), True, out=top)
        attn_ws = self._workspace("attn_bwd", _lib.query("gptrig_attn_bwd_workspace_bytes", Bm, H, S, D))
        rope_c, rope_s = rope_tables(S, D, self.device)
        for i in reversed(range(c.layers)):
            p = f"blocks/{i}/"
            x_in, xn1, rstd1, qkv, o, lse, x1, xn2, rstd2, mlp_state = saved.pop()
            if unit:
                dm = dx  # (dense) already written into this layer's down-projection gradient rows
            elif c.experts:
                dm = (dx * self.residual_scale).to(BF16)
            else:
                dm = lin_dout[i]["mlp_down"]
                dm.copy_((dx * self.residual_scale).to(BF16))
            if c.experts:
                dxn2 = self._routed_backward(p, xn2, mlp_state, dm)
            else:
                h, _ = mlp_state
                dg = torch.mm(dm, A.w(p + "mlp_down_w").t())
                dh = lin_dout[i]["mlp_up"]
                _lib.call("gptrig_bias_gelu_bwd", dg.data_ptr(), h.data_ptr(), A.w(p + "mlp_up_b").data_ptr(),
                          dh.data_ptr(), dh.shape[0], dh.shape[1], stream)
                dxn2 = torch.mm(dh, A.w(p + "mlp_up_w").t())
            dx1, _ = rmsnorm_backward(dxn2, x1, A.w(p + "ln2_scale"), rstd2, A.grad(p + "ln2_scale"), True,
                                      dresidual=dx, out=lin_dout[i]["attn"] if unit else None)
            if unit:
                da = dx1
            else:
                da = lin_dout[i]["attn"]
                da.copy_((dx1 * self.residual_scale).to(BF16))
            do = torch.mm(da, A.w(p + "attn_w").t())
            dqkv = lin_dout[i]["qkv"]
            # Attention backward with the RoPE VJP of q and k fused into its
            # dq / dk epilogues.
            with self._timed("attn_bwd"):
                _lib.call("gptrig_attn_bwd_rope", qkv.data_ptr(), qkv[:, d:].data_ptr(), qkv[:, 2 * d:].data_ptr(),
                          o.data_ptr(), do.data_ptr(), lse.data_ptr(), _lib.ptr(seg), dqkv.data_ptr(),
                          dqkv[:, d:].data_ptr(), dqkv[:, 2 * d:].data_ptr(), attn_ws.data_ptr(), attn_ws.numel(),
                          Bm, H, S, D, bwd_strides.data_ptr(), self.scale, rope_c.data_ptr(), rope_s.data_ptr(),
                          stream)
            if mark_layers:  # this layer's four output-gradients are written
                self._layer_ready[i].record()
            dxn1 = torch.mm(dqkv, A.w(p + "qkv_w").t())
            below = lin_dout[i - 1]["mlp_down"] if (unit and i > 0 and not c.experts) else None
            dx, _ = rmsnorm_backward(dxn1, x_in, A.w(p + "ln1_scale"), rstd1, A.grad(p + "ln1_scale"), True,
                                     dresidual=dx1, out=below)
        _lib.call("gptrig_embedding_bwd", tok.data_ptr(), dx.data_ptr(), A.grad("token_embedding").data_ptr(), N, d,
                  c.vocab_size, stream)

    def _weight_grad(self, prefix: str, inp: torch.Tensor, dout: torch.Tensor) -> None:
        """dW += inp^T dout and db += sum_rows(dout), both float32."""

        A = self.arena
        n, rows_in = inp.shape
        _lib.call("gptrig_weight_grad", inp.data_ptr(), dout.data_ptr(), A.grad(prefix + "_w").data_ptr(),
                  A.grad(prefix + "_b").data_ptr(), n, rows_in, dout.shape[1], _lib.stream())

    # -- the step ----------------------------------------------------------------------
    def train_step(self, x: torch.Tensor, y: torch.Tensor) -> None:
        """One optimizer step on a global batch ``x, y`` (int32 ``[batch, seq]``).

        Everything stays on the device; ``history`` row ``step-1`` receives
        ``(loss, lr, grad_norm)`` (``train.py:1446-1447``).
        """

        c = self.config
        A = self.arena
        stream = _lib.stream()
        A.g.zero_()
        self.loss.zero_()
        if tuple(x.shape) != (c.batch_size, c.seq_len) or tuple(y.shape) != (c.batch_size, c.seq_len):
            raise ValueError(f"train_step takes [batch_size, seq_len] = [{c.batch_size}, {c.seq_len}] tokens, got "
                             f"{tuple(x.shape)} / {tuple(y.shape)}")
        mb = c.micro_batch_size
        n_micro = x.shape[0] // mb
        weight = 1.0 / (n_micro * mb * x.shape[1])
        for j in range(n_micro):
            self._forward_backward(x[j * mb:(j + 1) * mb], y[j * mb:(j + 1) * mb], weight, j,
                                   mark_layers=j == n_micro - 1)
        # Weight gradients on the second stream, each layer after its event
        # (the layers finish top-down).  They write only the block linears'
        # gradient rows, which nothing on the main stream touches until the
        # optimizer update.
        main = torch.cuda.current_stream(self.device)
        side = self.wgrad_stream
        for i in reversed(range(c.layers)):
            side.wait_event(self._layer_ready[i])
            with torch.cuda.stream(side):
                for name in self.linears:
                    self._weight_grad(f"blocks/{i}/{name}", self.lin_in[i][name], self.lin_dout[i][name])
        main.wait_stream(side)
        self.step_count += 1
        step = self.step_count
        lr = learning_rate(step, c.optimizer)
        row = self.history[step - 1] if step <= self.history.shape[0] else None
        with self._timed("adamw"):
            if c.optimizer.grad_clip > 0.0:
                _lib.call("gptrig_sq_norm_partials", A.g.data_ptr(), A.n_chunks, CHUNK, self.sq_partials.data_ptr(),
                          stream)
                _lib.call("gptrig_finalize_norm", self.sq_partials.data_ptr(), A.n_chunks, c.optimizer.grad_clip,
                          self.norm.data_ptr(), self.clip.data_ptr(), self.loss.data_ptr(), lr,
                          _lib.ptr(row), stream)
                _lib.call("gptrig_adamw", A.p.data_ptr(), A.g.data_ptr(), A.m.data_ptr(), A.v.data_ptr(),
                          A.shadow.data_ptr(), A.chunk_tensor.data_ptr(), self.hparams.data_ptr(), A.n_chunks, CHUNK,
                          lr, self.beta1, self.beta2, step, self.clip.data_ptr(), None, stream)
            else:
                _lib.call("gptrig_adamw", A.p.data_ptr(), A.g.data_ptr(), A.m.data_ptr(), A.v.data_ptr(),
                          A.shadow.data_ptr(), A.chunk_tensor.data_ptr(), self.hparams.data_ptr(), A.n_chunks, CHUNK,
                          lr, self.beta1, self.beta2, step, None, self.sq_partials.data_ptr(), stream)
                _lib.call("gptrig_finalize_norm", self.sq_partials.data_ptr(), A.n_chunks, 0.0, self.norm.data_ptr(),
                          None, self.loss.data_ptr(), lr, _lib.ptr(row), stream)
            A.refresh_transposed()

    def eval_step(self, x: torch.Tensor, y: torch.Tensor, mask: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Masked loss sum and target count (``eval_step``, ``train.py:1493-1525``, tiled loss).

        ``x``, ``y``: int32 ``[batch, seq_len]`` tokens and targets, ``batch`` a
        multiple of ``micro_batch_size`` up to ``batch_size``; ``mask`` the same
        shape, any dtype (cast to float32).  Returns ``(sum(losses * mask),
        sum(mask))`` as float32 device scalars, without a host sync.
        """

        c = self.config
        shape = tuple(x.shape)
        mb = c.micro_batch_size
        if (len(shape) != 2 or shape[1] != c.seq_len or shape[0] % mb or shape[0] > c.batch_size
                or tuple(y.shape) != shape or tuple(mask.shape) != shape):
            raise ValueError(f"eval_step takes [k * {mb} <= {c.batch_size}, {c.seq_len}] tokens, targets and mask, "
                             f"got {shape} / {tuple(y.shape)} / {tuple(mask.shape)}")
        stream = _lib.stream()
        out = torch.zeros(2, dtype=F32, device=self.device)
        weights = mask.to(device=self.device, dtype=F32).contiguous()
        head = self.arena.w(self.head_path)
        for j in range(shape[0] // mb):
            tokens = x[j * mb:(j + 1) * mb]
            _, _, _, xf, _, _ = self._forward(tokens, j)
            n = tokens.numel()
            tgt = y[j * mb:(j + 1) * mb].reshape(-1).to(torch.int32).contiguous()
            losses = torch.empty(n, dtype=F32, device=self.device)
            lse = torch.empty(n, dtype=F32, device=self.device)
            ws = self._workspace("flce_fwd", _lib.query("gptrig_flce_fwd_workspace_bytes", n, c.d_model,
                                                        c.vocab_size))
            _lib.call("gptrig_flce_fwd", xf.data_ptr(), head.data_ptr(), tgt.data_ptr(), losses.data_ptr(),
                      lse.data_ptr(), ws.data_ptr(), ws.numel(), n, c.d_model, c.vocab_size,
                      c.semantic_vocab_size, stream)
            _lib.call("gptrig_masked_sum", losses.data_ptr(), weights[j * mb:(j + 1) * mb].data_ptr(), n,
                      out.data_ptr(), stream)
        return out[0], out[1]

    def history_rows(self) -> np.ndarray:
        """Copy the on-device ``(loss, lr, grad_norm)`` history (one sync)."""

        return self.history[: self.step_count].cpu().numpy()

    def write_training_log(self, output_dir, flops_per_token: float | None = None):
        """Persist the curve so far as ``training.riglog`` (``rig/runlog.py:257-302``,
        called once after the loop in ``train.py``); returns its path."""

        from . import runlog

        steps = min(self.step_count, self.history.shape[0])
        return runlog.write_training_log(output_dir, self.history[:steps].cpu().numpy(),
                                         tokens_per_step=self.config.batch_size * self.config.seq_len,
                                         final_step=steps, flops_per_token=flops_per_token)
