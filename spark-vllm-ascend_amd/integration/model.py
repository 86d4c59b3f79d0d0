"""Batch-1 decode of a Q4_0 decoder, one captured HIP graph per step.

The reference replaces every decode step of every layer with one compiled
kernel launch, ``layer_run(x, residual, positions, layer_name) -> (y,
residual)`` (src/spark_vllm_ascend/integration/model.py:46-80), called by
the model loop after the first input norm (src/spark_vllm_ascend/plugin/
spark2_5.py:369-376), with the last layer's "next norm" being the model's
final norm (integration/model.py:88-92).  vLLM captures the whole step in
one device graph (src/tools/deployment/serve.py:34).

Here one decode step is the kernel sequence (fused=True, the default)

  per layer:  add + RMSNorm(input_norm) fused into the QKV Q4_0 GEMV
              -> q/k RMSNorm + RoPE + KV write fused into split-KV attention
              -> LSE merge -> o_proj Q4_0 GEMV
              -> add + RMSNorm(post_attention_norm) fused into the gate|up
                 Q4_0 GEMV with SwiGLU -> down Q4_0 GEMV
  add + RMSNorm(final norm) fused into the head Q4_0 GEMV, whose workgroups
  also leave per-workgroup argmax keys -> on-device advance (reduces the keys
  to the next input id; position, sequence length, KV slot; gathers the next
  id's embedding row, the input of the next step)

i.e. 6 launches per layer.  Each layer hands (down output, residual) to the
next, whose first GEMV adds and normalises them (the reference's "next norm"
at the end of a layer, moved to the consumer).  fused=False runs the same
math as separate launches (add_rmsnorm, GEMV, q/k-norm kernel, attention,
argmax), 9 per layer.

captured once as a torch.cuda.CUDAGraph (a hipGraph).  Position, sequence
length and slot are read from device memory by the kernels, as the
reference reads them with load_bypass (src/spark_vllm_ascend/kernels/
layer.py:52-53), so one graph serves every step; prompt tokens are fed
through the same graph by the advance kernel's forced-id table.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from ..native import torch_ops
from .attention import choose_num_splits, choose_plan
from .head import TiedQ4_0Head
from .linear import Q4_0Linear, gemm_weight
from .weights import synthetic_q4_0


@dataclass
class DecoderConfig:
    hidden: int = 2560
    n_layers: int = 36
    n_q: int = 32
    n_kv: int = 8
    head_dim: int = 128
    intermediate: int = 9728
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    block_size: int = 128
    # gate/up activation: "swiglu" (silu(g) * u) or "gelu", the reference
    # model's erf-GELU(g) * u through its bf16 table (src/spark_vllm_ascend/
    # kernels/linear.py:540-577, table at integration/model.py:13-16)
    activation: str = "swiglu"

    @property
    def qkv_rows(self) -> int:
        return (self.n_q + 2 * self.n_kv) * self.head_dim


def rope_cos_sin_cache(max_position: int, rot_dim: int, theta: float, device) -> torch.Tensor:
    """vLLM's rotary table: inv_freq = theta^(-2i/d) in fp32, angles =
    pos * inv_freq, rows cos | sin, cast to the model dtype (bf16)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, rot_dim, 2, dtype=torch.float32) / rot_dim))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).to(torch.bfloat16).to(device)


def _norm_weight(n: int, gen: torch.Generator, device) -> torch.Tensor:
    return (1.0 + 0.1 * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16)


@dataclass
class DecoderLayer:
    qkv: Q4_0Linear
    o_proj: Q4_0Linear
    gate_up: Q4_0Linear
    down: Q4_0Linear
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    kv_cache: torch.Tensor  # [2, num_blocks, block_size, n_kv, head_dim]
    name: str = ""


@dataclass
class DecodeState:
    """Device-resident step inputs (graph-invariant addresses)."""
    ids: torch.Tensor            # int64 [1]
    positions: torch.Tensor      # int64 [1]
    seq_lens: torch.Tensor       # int32 [1]
    slot_mapping: torch.Tensor   # int64 [1]
    block_table: torch.Tensor    # int32 [1, max_blocks]
    next_ids: torch.Tensor       # int64 [1]
    forced: torch.Tensor         # int64 [1, max_len] prompt / teacher tokens
    forced_len: torch.Tensor     # int32 [1]: positions below it take forced tokens
    tokens: torch.Tensor         # int64 [1, max_len] every token fed, by position


class DecodeModel:
    """A Q4_0 decoder with random-init weights of a given shape, decoding
    `batch` sequences per step (one token each).  batch == 1 runs the fused
    GEMV path; batch > 1 runs the MFMA Q4_0 GEMM (m = batch rows; over the
    packed weight layout unless packed=False) with separate add+RMSNorm
    launches and the fused q/k-norm + RoPE + KV-write
    split-KV kernel over a per-sequence split plan (one plan launch per
    step), over a block table with one row per sequence."""

    def __init__(self, cfg: DecoderConfig, device, seed: int = 0, max_len: int = 8192,
                 num_splits: int | None = None, weights: dict | None = None,
                 fused: bool = True, batch: int = 1, plan_items: int | None = None,
                 packed: bool = True):
        if not 1 <= batch <= 16:
            raise ValueError("batch must be in [1, 16]")
        if cfg.activation not in ("swiglu", "gelu"):
            raise ValueError(f"activation must be 'swiglu' or 'gelu', got {cfg.activation!r}")
        self.cfg = cfg
        self.batch = B = batch
        self.fused = fused and batch == 1
        self.device = torch.device(device)
        self.max_len = max_len
        c = cfg
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        blocks_per_seq = -(-max_len // c.block_size)
        self.num_blocks = B * blocks_per_seq + 1
        self.layers: list[DecoderLayer] = []
        for i in range(c.n_layers):
            s = seed * 1000 + i * 10
            qkv = Q4_0Linear(c.hidden, [c.n_q * c.head_dim, c.n_kv * c.head_dim,
                                        c.n_kv * c.head_dim], device=self.device)
            o_proj = Q4_0Linear(c.n_q * c.head_dim, [c.hidden], device=self.device)
            gate_up = Q4_0Linear(c.hidden, [c.intermediate, c.intermediate], device=self.device)
            down = Q4_0Linear(c.intermediate, [c.hidden], device=self.device)
            for j, lin in enumerate((qkv, o_proj, gate_up, down)):
                key = f"layers.{i}.{('qkv', 'o_proj', 'gate_up', 'down')[j]}"
                if weights is not None and key in weights:
                    lin.qweight.data.copy_(weights[key])
                else:
                    lin.qweight.data.copy_(synthetic_q4_0(lin.q4_0_n, lin.q4_0_k, s + j,
                                                          self.device))
                lin.quant_method.process_weights_after_loading(lin)
            norms = []
            for j, n in enumerate((c.hidden, c.hidden, c.head_dim, c.head_dim)):
                key = f"layers.{i}.norm{j}"
                norms.append(weights[key].to(self.device) if weights is not None and key in weights
                             else _norm_weight(n, gen, self.device))
            kv = torch.zeros((2, self.num_blocks, c.block_size, c.n_kv, c.head_dim),
                             dtype=torch.bfloat16, device=self.device)
            self.layers.append(DecoderLayer(qkv, o_proj, gate_up, down, *norms, kv_cache=kv,
                                            name=f"model.layers.{i}.self_attn.attn"))
        self.final_norm = (weights["final_norm"].to(self.device)
                           if weights is not None and "final_norm" in weights
                           else _norm_weight(c.hidden, gen, self.device))
        head_blocks = (weights["head"] if weights is not None and "head" in weights
                       else synthetic_q4_0(c.vocab, c.hidden, seed * 1000 + 999, self.device))
        self.head = TiedQ4_0Head(head_blocks.to(self.device), c.vocab, c.hidden)
        # batch > 1: the MFMA GEMMs read the packed layout (torch_ops.q4_0_repack;
        # layers whose K is not a multiple of 256 keep the GGUF GEMM); the
        # one-row GEMVs and the embedding keep reading the GGUF blocks
        self.head_packed = None
        if batch > 1 and packed:
            for L in self.layers:
                for lin in (L.qkv, L.o_proj, L.down):
                    lin.quant_method.pack(lin)
                L.gate_up.quant_method.pack(L.gate_up, gated=True)
            if c.hidden % 256 == 0:
                self.head_packed = torch_ops.q4_0_repack(self.head.q4_0_head.view(-1), c.vocab,
                                                         c.hidden)
        self.cos_sin = rope_cos_sin_cache(max_len, c.head_dim, c.rope_theta, self.device)
        # the GELU table the gate/up epilogues read (None: SwiGLU)
        self.act_lut = torch_ops.gelu_table(self.device) if c.activation == "gelu" else None
        self.scale = 1.0 / math.sqrt(c.head_dim)
        if B == 1:
            self.num_items = 0
            self.num_splits = num_splits or choose_num_splits(blocks_per_seq * c.block_size)
        else:
            items, splits = choose_plan(B, c.n_kv)
            self.num_items = plan_items or items
            self.num_splits = num_splits or splits

        # pages are handed out in a seeded shuffled order, to exercise paging
        perm = torch.randperm(self.num_blocks, generator=torch.Generator().manual_seed(seed))
        table = perm[:B * blocks_per_seq].to(torch.int32).view(B, -1)
        dev = self.device
        self.state = DecodeState(
            ids=torch.zeros(B, dtype=torch.int64, device=dev),
            positions=torch.zeros(B, dtype=torch.int64, device=dev),
            seq_lens=torch.ones(B, dtype=torch.int32, device=dev),
            slot_mapping=torch.zeros(B, dtype=torch.int64, device=dev),
            block_table=table.to(dev),
            next_ids=torch.zeros(B, dtype=torch.int64, device=dev),
            forced=torch.zeros((B, max_len), dtype=torch.int64, device=dev),
            forced_len=torch.zeros(B, dtype=torch.int32, device=dev),
            tokens=torch.full((B, max_len), -1, dtype=torch.int64, device=dev),
        )
        # activations (fixed addresses for graph capture)
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.x = torch.empty((B, c.hidden), **bf)         # embedding of the input id
        self.res_a = torch.empty((B, c.hidden), **bf)     # residual after the attention add
        self.res_b = torch.empty((B, c.hidden), **bf)     # residual after the MLP add
        self.d = torch.empty((B, c.hidden), **bf)         # down projection output
        self.h = torch.empty((B, c.hidden), **bf)         # normalised input (unfused)
        self.qkv_out = torch.empty((B, c.qkv_rows), **bf)
        self.q = torch.empty((B, c.n_q, c.head_dim), **bf)
        self.attn = torch.empty((B, c.n_q, c.head_dim), **bf)
        self.o = torch.empty((B, c.hidden), **bf)
        self.h2 = torch.empty((B, c.hidden), **bf)
        self.act = torch.empty((B, c.intermediate), **bf)
        self.logits = torch.empty((B, c.vocab), **bf)
        self.partial_o = torch.empty((B, self.num_splits, c.n_q, c.head_dim), dtype=torch.float32,
                                     device=dev)
        self.partial_lse = torch.empty((B, self.num_splits, c.n_q), dtype=torch.float32, device=dev)
        self.plan = (torch.empty((self.num_items + B, torch_ops.PLAN_WORDS), dtype=torch.int32,
                                 device=dev) if self.num_items else None)
        # greedy-argmax keys: the head GEMV's (one row) or the head GEMM's
        nk = (torch_ops.argmax_keys_size(c.vocab, c.hidden) if B == 1
              else torch_ops.gemm_keys_per_row(c.vocab))
        self.argmax_keys = (torch.empty((B, nk), dtype=torch.int64, device=dev) if nk > 0
                            else None)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.runner = None  # native.runner.StepRunner after record_runner()

    @classmethod
    def from_gguf(cls, path, device, max_len: int = 8192, num_splits: int | None = None,
                  block_size: int = 128, fused: bool = True,
                  activation: str = "swiglu", batch: int = 1,
                  packed: bool = True) -> "DecodeModel":
        """A model whose weights come from a local GGUF file (Q4_0 linears and
        head, float norms rounded to bf16), shapes from its metadata.  GGUF
        metadata does not name the gate activation, so it is an argument:
        "swiglu" (the 4B Q4_0 decoder) or "gelu", the reference model's
        table erf-GELU (src/spark_vllm_ascend/integration/model.py:13-16).
        batch / packed: as for the constructor (batch > 1 decodes that many
        sequences per step, over the packed weight layout unless packed is
        False)."""
        from .gguf_file import GGUFFile, decoder_config, decoder_weights
        if activation not in ("swiglu", "gelu"):
            raise ValueError(f"activation must be 'swiglu' or 'gelu', got {activation!r}")
        g = GGUFFile(path)
        cfg = DecoderConfig(**decoder_config(g), block_size=block_size, activation=activation)
        dev = torch.device(device)
        w = {}
        for k, v in decoder_weights(g, cfg.n_layers).items():
            t = torch.from_numpy(v.copy())
            w[k] = (t.to(torch.bfloat16) if t.dtype == torch.float32 else t).to(dev)
        return cls(cfg, dev, max_len=max_len, num_splits=num_splits, weights=w, fused=fused,
                   batch=batch, packed=packed)

    # ------------------------------------------------------------------ step
    def _layer_input(self, i: int):
        """(activation, residual) entering layer i: the embedding alone for
        layer 0, else the previous layer's down output and residual."""
        return (self.x, None) if i == 0 else (self.d, self.res_b)

    def layer_run(self, i: int) -> None:
        """Decoder layer i: reads _layer_input(i), leaves the down projection
        in self.d and the residual stream in self.res_b (the next consumer
        adds and normalises them)."""
        c, L, st = self.cfg, self.layers[i], self.state
        ops = torch_ops
        x_in, r_in = self._layer_input(i)
        if self.fused:
            ops.add_rmsnorm_gemv(x_in, r_in, L.input_norm, L.qkv.qweight, c.qkv_rows, c.hidden,
                                 c.eps, residual_out=self.res_a, out=self.qkv_out)
            ops.qknorm_rope_splitkv_decode_merged(
                self.qkv_out, L.q_norm, L.k_norm, self.cos_sin, st.positions, st.slot_mapping,
                L.kv_cache[0], L.kv_cache[1], st.block_table, st.seq_lens, self.num_splits,
                self.scale, c.eps, c.n_q, self.partial_o, self.partial_lse, out=self.attn)
            ops.q4_0_gemv(self.attn, L.o_proj.qweight, c.hidden, c.n_q * c.head_dim, out=self.o)
            ops.add_rmsnorm_gemv_swiglu(self.o, self.res_a, L.post_norm, L.gate_up.qweight,
                                        c.intermediate, c.hidden, c.eps, residual_out=self.res_b,
                                        out=self.act, lut=self.act_lut)
        elif self.batch > 1:
            B = self.batch
            ops.add_rmsnorm(x_in, r_in, L.input_norm, c.eps, out=self.h, residual_out=self.res_a)
            ops.q4_0_gemm(self.h, gemm_weight(L.qkv), c.qkv_rows, c.hidden, out=self.qkv_out)
            ops.qknorm_rope_splitkv_decode_planned_merged(
                self.qkv_out, L.q_norm, L.k_norm, self.cos_sin, L.kv_cache[0], L.kv_cache[1],
                st.block_table, self.plan, self.num_items, self.scale, c.eps, c.n_q,
                self.partial_o, self.partial_lse, out=self.attn)
            ops.q4_0_gemm(self.attn.view(B, -1), gemm_weight(L.o_proj), c.hidden,
                          c.n_q * c.head_dim, out=self.o)
            ops.add_rmsnorm(self.o, self.res_a, L.post_norm, c.eps, out=self.h2,
                            residual_out=self.res_b)
            ops.q4_0_gemm_swiglu(self.h2, gemm_weight(L.gate_up, gated=True), c.intermediate,
                                 c.hidden, out=self.act, lut=self.act_lut)
            ops.q4_0_gemm(self.act, gemm_weight(L.down), c.hidden, c.intermediate, out=self.d)
            return
        else:
            ops.add_rmsnorm(x_in, r_in, L.input_norm, c.eps, out=self.h, residual_out=self.res_a)
            ops.q4_0_gemv(self.h, L.qkv.qweight, c.qkv_rows, c.hidden, out=self.qkv_out)
            ops.qknorm_rope_kv_write(self.qkv_out, L.q_norm, L.k_norm, self.cos_sin, st.positions,
                                     st.slot_mapping, L.kv_cache[0], L.kv_cache[1], c.n_q, c.n_kv,
                                     c.eps, q_out=self.q)
            ops.splitkv_decode_merged(self.q, L.kv_cache[0], L.kv_cache[1], st.block_table,
                                      st.seq_lens, self.num_splits, self.scale, self.partial_o,
                                      self.partial_lse, out=self.attn)
            ops.q4_0_gemv(self.attn, L.o_proj.qweight, c.hidden, c.n_q * c.head_dim, out=self.o)
            ops.add_rmsnorm(self.o, self.res_a, L.post_norm, c.eps, out=self.h2,
                            residual_out=self.res_b)
            if self.act_lut is None:
                ops.q4_0_gemv_swiglu(self.h2, L.gate_up.qweight, c.intermediate, c.hidden,
                                     out=self.act)
            else:
                ops.q4_0_gemv_gelu(self.h2, L.gate_up.qweight, self.act_lut, c.intermediate,
                                   c.hidden, out=self.act)
        ops.q4_0_gemv(self.act, L.down.qweight, c.hidden, c.intermediate, out=self.d)

    def enqueue_step(self) -> None:
        c, st = self.cfg, self.state
        ops = torch_ops
        # self.x holds the embedding of st.ids: gathered by the previous
        # step's advance kernel, or by reset() / set_context()
        if self.plan is not None:
            # this step's splits from the lengths / positions / slots the
            # previous advance left; every layer's attention reads them
            ops.splitkv_plan(st.seq_lens, st.block_table, c.block_size, self.num_items,
                             self.partial_o, self.partial_lse, positions=st.positions,
                             slot_mapping=st.slot_mapping, plan=self.plan)
        for i in range(len(self.layers)):
            self.layer_run(i)
        x_in, r_in = self._layer_input(len(self.layers))
        keys = None
        if self.fused and self.argmax_keys is not None:
            ops.add_rmsnorm_gemv_argmax(x_in, r_in, self.final_norm, self.head.q4_0_head,
                                        c.vocab, c.hidden, c.eps, self.argmax_keys.view(-1),
                                        out=self.logits)
            keys = self.argmax_keys
        elif self.batch > 1 and self.argmax_keys is not None:
            # the final norm's residual output is unused: res_a (free after
            # the last layer's post norm) takes it, so the step allocates
            # nothing (a recorded step must not, see record_runner)
            ops.add_rmsnorm(x_in, r_in, self.final_norm, c.eps, out=self.h,
                            residual_out=self.res_a)
            head = self.head_packed if self.head_packed is not None else self.head.q4_0_head
            ops.q4_0_gemm_argmax(self.h, head, c.vocab, c.hidden, self.argmax_keys,
                                 out=self.logits)
            keys = self.argmax_keys
        else:
            ops.add_rmsnorm(x_in, r_in, self.final_norm, c.eps, out=self.h,
                            residual_out=self.res_a)
            ops.q4_0_gemv(self.h, self.head.q4_0_head, c.vocab, c.hidden, out=self.logits)
            ops.argmax(self.logits, out=st.next_ids)
        ops.decode_advance(st.next_ids, st.ids, st.positions, st.seq_lens, st.slot_mapping,
                           st.block_table, c.block_size, tokens_out=st.tokens,
                           forced_ids=st.forced, forced_len=st.forced_len, argmax_keys=keys,
                           embed_table=self.head.weight, embed_out=self.x)

    def capture(self) -> None:
        """Capture one decode step as a graph.  Clobbers the decode state;
        call reset() afterwards."""
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.enqueue_step()  # warm-up outside the graph
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.enqueue_step()
        self.graph = g

    def record_runner(self, runner=None):
        """Record one decode step into a step runner (native/runner.py): the
        counterpart of capture() that replays the step's kernels as AQL
        dispatch packets on a queue of the library's own.  Recording launches
        nothing and leaves the decode state as it is."""
        from ..native.runner import StepRunner
        self.runner = runner if runner is not None else StepRunner()
        self.runner.record(self.enqueue_step)
        return self.runner

    def run_steps(self, n: int, fences: str = "agent", timeout_s: float = 60.0) -> None:
        """n decode steps through the recorded runner, waiting for them."""
        if self.runner is None:
            raise RuntimeError("record_runner() first")
        self.runner.run(n, fences, timeout_s)

    def step(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            self.enqueue_step()

    # --------------------------------------------------------------- control
    def reset(self, prompt) -> None:
        """Position 0 of each sequence holds its prompt[0]; the advance kernel
        feeds the remaining prompt tokens, then the model's own argmax.
        prompt: a 1-D tensor (batch 1, or the same prompt for every sequence)
        or a list of `batch` 1-D tensors (prompts of any lengths)."""
        st = self.state
        B = self.batch
        prompts = list(prompt) if isinstance(prompt, (list, tuple)) else [prompt] * B
        if len(prompts) != B:
            raise ValueError(f"need {B} prompts")
        st.forced.zero_()
        st.tokens.fill_(-1)
        lens = []
        for r, p in enumerate(prompts):
            seq = torch.as_tensor(p).to(device=self.device, dtype=torch.int64).view(-1)
            if not 1 <= seq.numel() <= self.max_len:
                raise ValueError("a prompt must have 1..max_len tokens")
            st.forced[r, :seq.numel()] = seq
            st.tokens[r, 0] = seq[0]
            st.ids[r] = seq[0]
            lens.append(seq.numel())
        st.forced_len.copy_(torch.tensor(lens, dtype=torch.int32))
        st.positions.zero_()
        st.seq_lens.fill_(1)
        st.slot_mapping.copy_(st.block_table[:, 0].to(torch.int64) * self.cfg.block_size)
        self.head.embed(st.ids, out=self.x)

    def fill_kv(self, seed: int) -> None:
        """Seeded N(0, 1) bf16 values in every layer's whole KV cache (K and V
        planes), generated on the device: a cache with realistic contents
        for decoding at a given context after set_context()."""
        g = torch.Generator(device=self.device).manual_seed(seed)
        for L in self.layers:
            L.kv_cache.normal_(0.0, 1.0, generator=g)

    def set_context(self, lengths, ids=None) -> None:
        """Continue every sequence r at position lengths[r] (the KV cache
        below it is whatever it holds): for timing decode at given contexts."""
        st = self.state
        L = torch.as_tensor(lengths, dtype=torch.int64).view(-1)
        if L.numel() != self.batch or int(L.min()) < 0 or int(L.max()) >= self.max_len:
            raise ValueError("one length per sequence, below max_len")
        st.forced_len.zero_()
        st.positions.copy_(L)
        st.seq_lens.copy_((L + 1).to(torch.int32))
        bs = self.cfg.block_size
        rows = torch.arange(self.batch, device=self.device)
        Ld = L.to(self.device)
        st.slot_mapping.copy_(st.block_table[rows, Ld // bs].to(torch.int64) * bs + Ld % bs)
        st.ids.copy_(torch.as_tensor(ids if ids is not None else [1] * self.batch,
                                     dtype=torch.int64))
        self.head.embed(st.ids, out=self.x)

    def generate(self, prompt, new_tokens: int, fences: str | None = None) -> torch.Tensor:
        """Greedy decode: feeds the prompt(s), then new_tokens generated
        tokens.  Returns the token ids by position (prompt followed by
        generated): [total] for batch 1, else [batch, longest total].  With
        fences, the steps run on the recorded step runner (record_runner)
        with that fence mode, all of them in one replay."""
        prompts = list(prompt) if isinstance(prompt, (list, tuple)) else [prompt] * self.batch
        total = max(int(torch.as_tensor(p).numel()) for p in prompts) + new_tokens
        if total > self.max_len:
            raise ValueError("prompt + new_tokens exceeds max_len")
        self.reset(prompt)
        if fences is not None:
            if total > 1:
                self.run_steps(total - 1, fences)
        else:
            for _ in range(total - 1):
                self.step()
        torch.cuda.synchronize(self.device)
        out = self.state.tokens[:, :total].clone()
        return out[0] if self.batch == 1 else out
