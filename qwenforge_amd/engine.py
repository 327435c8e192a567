"""Greedy Qwen2-shaped decode engine around the HIP attention kernels.

Mirrors the reference's cached generation path without the tokenizer:

* ``prefill_ragged`` / ``generate_ragged`` -- ``_prefill_ragged``
  (SE:1162-1204) and the padded-batch decode of ``generate`` (SE:1241-1335)
  for variable-length prompts: rows packed along the token axis, one varlen
  prefill launch per layer, decode over the bias-masked holes.
* ``prefill`` -- ``StudentEngine._prefill`` (SE:679-737): per layer RMSNorm,
  fused QKV projection, then ONE fused HIP launch does rotate-half RoPE, the
  causal GQA attention and the KV-cache append (it replaces the eager RoPE
  SE:698-699/556-577, the slice append SE:715-716 and SDPA SE:719-725);
  o_proj, MLP, last-token logits.
* ``decode`` -- ``_decode_tokens_graphed`` (SE:984-1133) replaying a captured
  ``_decode_step_static`` (SE:876-982): per layer RMSNorm, QKV, the HIP
  RoPE+append kernel (SE:927-932), the HIP split-K decode attention bounded by
  the device-side write slot (SE:941-943), o_proj, MLP; final norm, lm_head,
  argmax.  The per-step bookkeeping the reference does on the host between
  replays (bias slot, write slot, positions, token store; SE:1126-1132) runs
  inside the graph as device ops, so a step is a single graph replay.
  Captured steps are kept per (batch, capacity, padded) in a ``GraphRegistry``
  (the reference's LRU registry under a 2.4 GB KV budget, SE:393-394 and
  SE:1090-1118): a later call of the same shape prefills into that entry's
  caches and only replays.

For batches of 1..4 rows the decode step body is the fused weight-streaming
path (``step_ops``, include/qf_step.h): per layer one launch for rms_norm +
QKV + RoPE + append, the split-K attention launch, one for the split merge +
o_proj + residual, one for rms_norm + gate/up + SwiGLU and one for down_proj +
residual; then one for rms_norm + lm_head + per-block argmax and one for the
argmax and the slot bookkeeping.  Larger batches keep the torch projections (hipBLASLt / ATen
kernels) around the same HIP attention kernels.  Prefill always uses the torch
projections.  Everything is fp16 storage with the reference's rounding points.
"""

from __future__ import annotations

from collections import OrderedDict

import torch
import torch.nn.functional as F

from . import ops, step_ops
from .model import Qwen2Config
from .rope import cos_sin, inv_freq


def cache_capacity(prompt_len: int, new_tokens: int, multiple: int = 64) -> int:
    """KV slots per row for a prompt of ``prompt_len`` tokens and ``new_tokens``
    greedy tokens on the graph path (SE:1263-1273): the prompt plus the
    ``new_tokens - 1`` decode steps that append (the last token is never fed
    back), at least the prompt, rounded up to ``multiple``."""
    cap = max(prompt_len + max(new_tokens - 1, 0), prompt_len)
    return (cap + multiple - 1) // multiple * multiple


class GraphRegistry:
    """Captured decode-step contexts, least recently used first.

    The reference keys them by (batch, capacity) and, after each capture,
    evicts the oldest entries while the persistent KV caches of all entries
    exceed a byte budget, never the entry just stored (SE:1090-1103, budget
    2.4 GB at SE:394); a hit moves the entry to the newest end (SE:1115-1118).
    """

    def __init__(self, byte_budget: int = 2_400_000_000):
        self.byte_budget = byte_budget
        self._entries: OrderedDict = OrderedDict()

    @staticmethod
    def kv_bytes(ctx) -> int:
        """Bytes of a context's per-layer K and V caches (SE:1094-1096)."""
        return sum(k.numel() * k.element_size() + v.numel() * v.element_size()
                   for k, v in ctx["caches"])

    def get(self, key):
        """The context stored under ``key`` (now the most recently used), or None."""
        ctx = self._entries.pop(key, None)
        if ctx is not None:
            self._entries[key] = ctx
        return ctx

    def put(self, key, ctx) -> None:
        """Store ``ctx`` as the most recently used entry, then evict the least
        recently used ones while the budget is exceeded."""
        self._entries.pop(key, None)
        self._entries[key] = ctx
        total = sum(self.kv_bytes(c) for c in self._entries.values())
        while total > self.byte_budget and len(self._entries) > 1:
            oldest = next(iter(self._entries))
            if oldest == key:
                break
            total -= self.kv_bytes(self._entries.pop(oldest))

    def clear(self) -> None:
        self._entries.clear()

    def keys(self) -> list:
        return list(self._entries)

    def __len__(self) -> int:
        return len(self._entries)


class DecodeEngine:
    """Batched greedy decoding of a Qwen2-shaped model on one MI355X."""

    def __init__(self, cfg: Qwen2Config, weights: dict, device="cuda", fused_step: bool = True,
                 tile_weights: bool = True):
        self.cfg = cfg
        self.device = torch.device(device)
        self.w = weights
        self.inv_freq = inv_freq(cfg.head_dim, cfg.rope_theta, self.device)
        self.scale = cfg.head_dim ** -0.5
        self.fused_step = fused_step
        self.tile_weights = tile_weights
        self._tiles = None
        self._lm_tiles = None
        self._o_tiles = None
        self._ctx = None
        self.graphs = GraphRegistry()
        self.captures = 0  # graph captures so far (registry hits capture nothing)

    # Rows from which the fused step reads the QKV and gate/up weights as
    # matrix-core tiles (batch rows as MFMA columns): measured on MI355X at
    # Qwen2.5-0.5B shape, 0.803 -> 0.756 ms per step at B=4, 0.672 -> 0.659 at
    # B=2, neutral at B=1 (the dot-product kernels stay there).
    TILE_MIN_BATCH = 2

    def projection_weights(self, i: int, batch: int):
        """(qkv, gate_up) weights of layer i for the fused step at ``batch``
        rows: row-major tensors, or their ``step_ops.Tiles`` (packed once, on
        first use; the row-major copies stay for prefill)."""
        layer = self.w["layers"][i]
        if not self.tile_weights or batch < self.TILE_MIN_BATCH:
            return layer["qkv_weight"], layer["gate_up_weight"]
        if self._tiles is None:
            self._tiles = [(step_ops.pack_weight(l["qkv_weight"], step_ops.PACK_ROPE),
                            step_ops.pack_weight(l["gate_up_weight"], step_ops.PACK_SWIGLU))
                           for l in self.w["layers"]]
        return self._tiles[i]

    def o_proj_weight(self, i: int, batch: int):
        """The o_proj weight of layer i for the fused step's merge + o_proj at
        ``batch`` rows: row-major, or its ``step_ops.Tiles`` from
        TILE_MIN_BATCH rows (packed once, on first use)."""
        w = self.w["layers"][i]["o_weight"]
        if not self.tile_weights or batch < self.TILE_MIN_BATCH or w.shape[0] % 16:
            return w
        if self._o_tiles is None:
            self._o_tiles = [step_ops.pack_weight(l["o_weight"], step_ops.PACK_PLAIN)
                             for l in self.w["layers"]]
        return self._o_tiles[i]

    # Rows from which the fused step's lm_head reads matrix-core tiles:
    # measured on MI355X at vocab 151936, 45.6-45.8 us per call at any batch
    # against the row kernel's 44.8 at B=2 and 51.1 at B=4.
    LM_TILE_MIN_BATCH = 3

    def lm_head_weight(self, batch: int):
        """The lm_head weight of the fused step at ``batch`` rows: row-major, or
        its ``step_ops.Tiles`` from LM_TILE_MIN_BATCH rows (packed once; the
        row-major copy stays the tied embedding and the prefill's head)."""
        w = self.w["lm_head"]
        if (not self.tile_weights or batch < self.LM_TILE_MIN_BATCH or w.shape[0] % 16
                or w.shape[1] % 32):
            return w
        if self._lm_tiles is None:
            self._lm_tiles = step_ops.pack_weight(w, step_ops.PACK_PLAIN)
        return self._lm_tiles

    def uses_fused_step(self, batch: int) -> bool:
        """The fused decode-step kernels cover 1..4 rows and hidden <= 1024."""
        return (self.fused_step and 1 <= batch <= step_ops.MAX_BATCH and self.cfg.hidden <= 1024
                and self.cfg.head_dim == step_ops.HEAD_DIM)

    # ------------------------------------------------------------------ helpers
    def _rms(self, x, weight):
        return F.rms_norm(x, (self.cfg.hidden,), weight, self.cfg.rms_eps)

    def _mlp(self, x, layer):
        gate, up = F.linear(x, layer["gate_up_weight"]).chunk(2, dim=-1)
        return F.linear(F.silu(gate) * up, layer["down_weight"])

    def _qkv(self, x, layer):
        cfg = self.cfg
        b, t, _ = x.shape
        projected = F.linear(x, layer["qkv_weight"], layer["qkv_bias"])
        q, k, v = projected.split((cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim,
                                   cfg.kv_heads * cfg.head_dim), dim=-1)
        q = q.view(b, t, cfg.heads, cfg.head_dim).transpose(1, 2)
        k = k.view(b, t, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
        v = v.view(b, t, cfg.kv_heads, cfg.head_dim).transpose(1, 2)
        return q, k, v

    # ------------------------------------------------------------------ prefill
    def new_caches(self, batch: int, capacity: int):
        """Zero-initialised (B, KVH, cap, D) caches, one pair per layer (SE:705-714)."""
        cfg = self.cfg
        shape = (batch, cfg.kv_heads, capacity, cfg.head_dim)
        return [(torch.zeros(shape, device=self.device, dtype=torch.float16),
                 torch.zeros(shape, device=self.device, dtype=torch.float16))
                for _ in range(cfg.layers)]

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, caches):
        """Equal-length prompts (B, S) -> last-token logits (B, vocab); fills the caches."""
        cfg = self.cfg
        b, s = input_ids.shape
        hidden = F.embedding(input_ids, self.w["embed"])
        cos, sin = cos_sin(torch.arange(s, device=self.device), self.inv_freq)
        for layer, (kc, vc) in zip(self.w["layers"], caches):
            residual = hidden
            q, k, v = self._qkv(self._rms(hidden, layer["input_norm"]), layer)
            att = ops.gqa_flash_prefill_rope_append(q, k, v, cos, sin, kc, vc, 0)
            att = att.transpose(1, 2).reshape(b, s, cfg.hidden)
            hidden = residual + F.linear(att, layer["o_weight"])
            residual = hidden
            hidden = residual + self._mlp(self._rms(hidden, layer["post_norm"]), layer)
        last = self._rms(hidden[:, -1], self.w["final_norm"])
        return F.linear(last, self.w["lm_head"])

    @torch.no_grad()
    def prefill_ragged(self, prompts, caches):
        """Variable-length prompts (a list of 1-D id tensors) -> last-token logits (B, vocab).

        ``_prefill_ragged`` (SE:1162-1204) runs ``_prefill`` once per row; here
        the rows are packed along the token axis, so every projection is one
        GEMM over all tokens and one varlen launch does RoPE, the cache append
        (slots [0, len_b) of row b) and the causal attention of every row.
        """
        return self._prefill_packed(
            prompts, lambda i, q, k, v, cu, n, cos, sin, lengths: ops.prefill_varlen(
                q, k, v, cu, n, cos, sin, caches[i][0], caches[i][1], 0, lengths=lengths))

    def _prefill_packed(self, prompts, attend):
        """Packed ragged prefill body; ``attend(layer, q, k, v, cu, max_len, cos,
        sin, lengths)`` runs the varlen RoPE + append + attention launch of one
        layer (``lengths``: the host row lengths ``cu`` was built from)."""
        cfg = self.cfg
        dev = self.device
        lengths = [int(p.numel()) for p in prompts]
        ids = torch.cat([p.reshape(-1).to(dev) for p in prompts])
        total = ids.numel()
        starts = [0]
        for n in lengths:
            starts.append(starts[-1] + n)
        cu = torch.tensor(starts, dtype=torch.int32, device=dev)
        pos = torch.cat([torch.arange(n, device=dev) for n in lengths])
        cos, sin = cos_sin(pos, self.inv_freq)                 # (T, D): each row's own positions
        qw, kvw = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        hidden = F.embedding(ids, self.w["embed"])
        for i, layer in enumerate(self.w["layers"]):
            residual = hidden
            proj = F.linear(self._rms(hidden, layer["input_norm"]), layer["qkv_weight"],
                            layer["qkv_bias"])
            q = proj[:, :qw].view(total, cfg.heads, cfg.head_dim)
            k = proj[:, qw:qw + kvw].view(total, cfg.kv_heads, cfg.head_dim)
            v = proj[:, qw + kvw:].view(total, cfg.kv_heads, cfg.head_dim)
            att = attend(i, q, k, v, cu, max(lengths), cos, sin, lengths)
            hidden = residual + F.linear(att.reshape(total, cfg.hidden), layer["o_weight"])
            residual = hidden
            hidden = residual + self._mlp(self._rms(hidden, layer["post_norm"]), layer)
        last = hidden[cu[1:].long() - 1]
        return F.linear(self._rms(last, self.w["final_norm"]), self.w["lm_head"])

    # ------------------------------------------------------------------ decode
    def _step(self, ctx):
        """One static-shape decode step (the captured graph body)."""
        if ctx.get("fused"):
            self._step_fused(ctx)
        else:
            self._step_torch(ctx)

    def _step_fused(self, ctx):
        """The step body on the fused weight-streaming kernels (B <= 4)."""
        cfg = self.cfg
        b = ctx["token"].shape[0]
        eps = cfg.rms_eps
        if ctx["bias"] is not None:
            ctx["bias"].index_fill_(1, ctx["write"], 0.0)
        # RoPE angles from the positions inside the QKV kernel: the same fp16
        # table as cos_sin (SE:910-915) without its separate launches.
        rope = (ctx["pos"], self.inv_freq)
        hidden, q_rot, h = ctx["hidden"], ctx["q_rot"], ctx["h"]
        for i, (layer, (kc, vc)) in enumerate(zip(self.w["layers"], ctx["caches"])):
            w_qkv, w_gate_up = self.projection_weights(i, b)
            if i == 0:
                # Embedding gather (SE:896) folded into the first projection.
                step_ops.rms_qkv_rope_append(self.w["embed"], layer["input_norm"], eps,
                                             w_qkv, layer["qkv_bias"], None, None,
                                             kc, vc, ctx["write"], q_rot, token=ctx["token"],
                                             hidden_out=hidden, positions=rope)
            else:
                step_ops.rms_qkv_rope_append(hidden, layer["input_norm"], eps, w_qkv,
                                             layer["qkv_bias"], None, None, kc, vc, ctx["write"],
                                             q_rot, positions=rope)
            grouped = q_rot.view(b, cfg.kv_heads, cfg.groups, cfg.head_dim)
            # Split-K partials; their merge is the o_proj kernel's prologue.
            # Without holes the splits cover the capacity (SE:851) with the
            # write slot as a mask: the cache is sized to the generation, so
            # few slots are read past it, and the first K/V loads need not
            # wait for it (measured per step: B=1 -0.6 us, B=4 -1.4 us; with
            # the ragged batch's bias +1.9 us, so that one splits the bound).
            ops.flash_decode_split(grouped, kc, vc, ctx["bias"], ctx["flash"],
                                   kv_last=ctx["write"], scale=self.scale,
                                   split_capacity=ctx["bias"] is None)
            step_ops.attn_merge_o_proj(ctx["flash"], self.o_proj_weight(i, b), hidden)
            step_ops.rms_gate_up_swiglu(hidden, layer["post_norm"], eps, w_gate_up, h)
            step_ops.gemv_residual(h, layer["down_weight"], hidden)
        step_ops.rms_lm_head(hidden, self.w["final_norm"], eps, self.lm_head_weight(b), ctx["logits"],
                             ctx["keys"])
        step_ops.argmax_step(ctx["keys"], ctx["token"], ctx["rows"], ctx["step"], ctx["write"],
                             ctx["pos"])

    def _step_torch(self, ctx):
        """The step body on torch projections around the HIP attention kernels."""
        cfg = self.cfg
        b = ctx["token"].shape[0]
        if ctx["bias"] is not None:
            # The slot written by this step becomes valid (SE:1127).
            ctx["bias"].index_fill_(1, ctx["write"], 0.0)
        hidden = F.embedding(ctx["token"], self.w["embed"]).view(b, 1, cfg.hidden)
        cos, sin = cos_sin(ctx["pos"], self.inv_freq)          # (B, D), once per step (SE:910-915)
        for layer, (kc, vc) in zip(self.w["layers"], ctx["caches"]):
            residual = hidden
            q, k, v = self._qkv(self._rms(hidden, layer["input_norm"]), layer)
            q_rot = ops.rope_append(q, k, v, cos, sin, kc, vc, ctx["write"])
            grouped = q_rot.view(b, cfg.kv_heads, cfg.groups, cfg.head_dim)
            att = ops.flash_decode_attention(grouped, kc, vc, ctx["bias"], ctx["flash"],
                                             kv_last=ctx["write"], scale=self.scale)
            hidden = residual + F.linear(att.reshape(b, 1, cfg.hidden), layer["o_weight"])
            residual = hidden
            hidden = residual + self._mlp(self._rms(hidden, layer["post_norm"]), layer)
        hidden = self._rms(hidden, self.w["final_norm"]).squeeze(1)
        logits = F.linear(hidden, self.w["lm_head"])
        nxt = torch.argmax(logits, dim=-1)
        ctx["logits"].copy_(logits)
        ctx["token"].copy_(nxt)
        ctx["rows"].index_copy_(1, ctx["step"], nxt.unsqueeze(1))
        ctx["write"].add_(1)
        ctx["pos"].add_(1)
        ctx["step"].add_(1)

    @staticmethod
    def fused_max_splits(batch: int) -> int:
        """Split cap of the fused step.  Every o_proj workgroup merges all splits
        of all rows, so that prologue's traffic grows with splits x rows;
        measured on MI355X at Qwen2.5-0.5B shape: 8 splits at B=1, 4 above."""
        return 8 if batch == 1 else 4

    def _flash_scratch(self, batch: int, cap: int):
        cfg = self.cfg
        if not self.uses_fused_step(batch):
            return ops.make_flash_scratch(batch, cfg.kv_heads, cfg.groups, cap, self.device)
        splits = min(ops.choose_splits(batch, cfg.kv_heads, cap), self.fused_max_splits(batch))
        return ops.make_flash_scratch(batch, cfg.kv_heads, cfg.groups, cap, self.device,
                                      splits=splits, fused=False)

    def make_context(self, caches, batch: int, max_new_tokens: int, bias_mask=None):
        """Static buffers of the graph step.  ``bias_mask`` (B, cap) bool marks
        valid prompt slots when rows are right-padded; None means no holes, so
        the write-slot bound alone selects the valid keys and no bias is read."""
        cfg = self.cfg
        cap = caches[0][0].shape[2]
        dev = self.device
        bias = None
        if bias_mask is not None:
            bias = torch.full((batch, cap), torch.finfo(torch.float16).min, device=dev,
                              dtype=torch.float16)
            bias.masked_fill_(bias_mask, 0.0)
        ctx = {
            "caches": caches,
            "bias": bias,
            "flash": self._flash_scratch(batch, cap),
            "token": torch.zeros(batch, device=dev, dtype=torch.long),
            "pos": torch.zeros(batch, device=dev, dtype=torch.long),
            "write": torch.zeros(1, device=dev, dtype=torch.long),
            "step": torch.zeros(1, device=dev, dtype=torch.long),
            "rows": torch.zeros(batch, max_new_tokens, device=dev, dtype=torch.long),
            "logits": torch.zeros(batch, cfg.vocab, device=dev, dtype=torch.float16),
            "fused": self.uses_fused_step(batch),
        }
        if ctx["fused"]:
            f16 = torch.float16
            ctx["hidden"] = torch.zeros(batch, cfg.hidden, device=dev, dtype=f16)
            ctx["q_rot"] = torch.zeros(batch, cfg.heads, cfg.head_dim, device=dev, dtype=f16)
            ctx["h"] = torch.zeros(batch, cfg.intermediate, device=dev, dtype=f16)
            ctx["keys"] = torch.zeros(batch, step_ops.lm_blocks(self.lm_head_weight(batch)),
                                      device=dev, dtype=torch.long)
        return ctx

    def capture(self, ctx):
        """Capture ``_step`` into a hipGraph (2 warm-ups on a side stream, SE:1056-1074).

        The warm-ups run with the write slot parked on the last cache slot, as
        in the reference; the caller resets the state before replaying.
        """
        cap = ctx["caches"][0][0].shape[2]
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        saved = {k: ctx[k].clone() for k in ("token", "pos", "write", "step", "rows")}
        with torch.cuda.stream(side):
            for _ in range(2):
                ctx["write"].fill_(cap - 1)
                ctx["step"].fill_(0)
                self._step(ctx)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            self._step(ctx)
        for k, v in saved.items():
            ctx[k].copy_(v)
        if ctx["bias"] is not None:
            ctx["bias"][:, cap - 1] = torch.finfo(torch.float16).min
        torch.cuda.synchronize(self.device)
        ctx["graph"] = graph
        self.captures += 1
        return graph

    # Fewest new tokens for which generate captures the step (SE:1274-1276):
    # shorter runs call the step eagerly, and a single token decodes nothing.
    GRAPH_MIN_NEW_TOKENS = 8

    def _graph_context(self, key, batch: int, cap: int, prefill, bias_mask=None,
                       capture: bool = True):
        """Run ``prefill(caches)`` into the registry entry ``key`` = (batch,
        cap, padded) and return (context, what prefill returned), capturing
        the step on a miss -- or, with ``capture`` False and no entry, into a
        fresh context that is neither captured nor stored.

        On a hit the prompt overwrites the entry's cache rows and the bias is
        rebuilt from ``bias_mask``; slots a previous call wrote past the new
        prompt are either masked by the bias (holes) or beyond the write slot,
        which bounds every attention read, and each decode step writes its
        slot before attending it (SE:1104-1114).  The rows buffer holds
        ``cap`` columns, the most new tokens a call of this capacity asks for.
        """
        ctx = self.graphs.get(key)
        caches = ctx["caches"] if ctx is not None else self.new_caches(batch, cap)
        result = prefill(caches)
        if ctx is None:
            ctx = self.make_context(caches, batch, cap, bias_mask=bias_mask)
            if capture:
                self.capture(ctx)
                self.graphs.put(key, ctx)
        elif bias_mask is not None:
            ctx["bias"].fill_(torch.finfo(torch.float16).min)
            ctx["bias"].masked_fill_(bias_mask, 0.0)
        return ctx, result

    def _replay_fn(self, ctx):
        """One decode step of ``ctx``: its graph's replay, or the step called
        eagerly when it was not captured (same results bit for bit)."""
        graph = ctx.get("graph")
        return graph.replay if graph is not None else (lambda: self._step(ctx))

    @torch.no_grad()
    def generate_ragged(self, prompts, max_new_tokens: int, timing: dict | None = None):
        """Greedy ids (B, max_new_tokens) for variable-length prompts (list of 1-D tensors).

        The reference's padded-batch semantics (SE:1241-1335): capacity =
        roundup64(max_len + new - 1); row b's prompt fills slots [0, len_b);
        decode step t writes the shared slot max_len + t - 1 at position
        len_b + t - 1, and the bias masks the holes [len_b, max_len).  Captured
        steps are reused per (batch, capacity) as in ``generate``.
        """
        b = len(prompts)
        lengths = [int(p.numel()) for p in prompts]
        p_max = max(lengths)
        cap = cache_capacity(p_max, max_new_tokens)
        mask = torch.zeros(b, cap, dtype=torch.bool, device=self.device)
        for i, n in enumerate(lengths):
            mask[i, :n] = True
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record()

        def run_prefill(caches):
            first = torch.argmax(self.prefill_ragged(prompts, caches), dim=-1)
            ev[1].record()
            return first

        ctx, first = self._graph_context((b, cap, True), b, cap, run_prefill, bias_mask=mask,
                                         capture=max_new_tokens >= self.GRAPH_MIN_NEW_TOKENS)
        ctx["rows"][:, 0] = first
        ctx["token"].copy_(first)
        ctx["pos"].copy_(torch.tensor(lengths, device=self.device))
        ctx["write"].fill_(p_max)
        ctx["step"].fill_(1)
        torch.cuda.synchronize(self.device)
        ev[2].record()
        step = self._replay_fn(ctx)
        for _ in range(1, max_new_tokens):
            step()
        ev[3].record()
        torch.cuda.synchronize(self.device)
        if timing is not None:
            timing["prefill_ms"] = ev[0].elapsed_time(ev[1])
            timing["decode_ms"] = ev[2].elapsed_time(ev[3])
        self._ctx = ctx
        return ctx["rows"][:, :max_new_tokens].clone()

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, timing: dict | None = None):
        """Greedy ids (B, max_new_tokens) for equal-length prompts (B, S).

        Capacity follows SE:1263-1273: prompt + new - 1, rounded up to 64.
        A call whose (batch, capacity) is in ``graphs`` reuses that captured
        step and its caches; below GRAPH_MIN_NEW_TOKENS new tokens a call that
        finds none runs the step eagerly instead of capturing it.  ``timing`` (optional dict) receives prefill and
        decode times in ms (HIP events on the current stream; a capture falls
        between the two and is in neither).
        """
        b, s = input_ids.shape
        cap = cache_capacity(s, max_new_tokens)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record()

        def run_prefill(caches):
            first = torch.argmax(self.prefill(input_ids, caches), dim=-1)
            ev[1].record()
            return first

        ctx, first = self._graph_context((b, cap, False), b, cap, run_prefill,
                                         capture=max_new_tokens >= self.GRAPH_MIN_NEW_TOKENS)
        ctx["rows"][:, 0] = first
        ctx["token"].copy_(first)
        ctx["pos"].fill_(s)
        ctx["write"].fill_(s)
        ctx["step"].fill_(1)
        torch.cuda.synchronize(self.device)
        ev[2].record()
        step = self._replay_fn(ctx)
        for _ in range(1, max_new_tokens):
            step()
        ev[3].record()
        torch.cuda.synchronize(self.device)
        if timing is not None:
            timing["prefill_ms"] = ev[0].elapsed_time(ev[1])
            timing["decode_ms"] = ev[2].elapsed_time(ev[3])
        self._ctx = ctx
        return ctx["rows"][:, :max_new_tokens].clone()
