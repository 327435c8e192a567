"""Greedy decoding over a paged KV cache, with continuous batching.

The reference pads a ragged batch to its longest prompt, shares one write
slot across rows and masks the holes with a bias (SE:1162-1204,
SE:1263-1335); "PagedAttention & Continuous Batching" is on its roadmap
(README.md:144).  ``PagedDecodeEngine`` runs the same model step over page
pools (``paged.PagedKvCache``):

* every row appends at its own slot (its current length) and attends over
  exactly its own slots, so no bias and no holes;
* a row only holds the pages its request needs;
* ``serve`` admits a waiting request into a row as soon as that row's request
  finishes: the row's pages go back to the pool, the new prompt is prefilled
  into fresh pages of the same row, and the captured step keeps replaying
  for all rows (first come, first served).

The captured step is the dense engine's step with the paged kernels: for 1..4
rows the fused weight-streaming kernels (QKV + RoPE + paged append, paged
split-K attention, merge + o_proj, gate/up, down, lm_head + argmax), above
that torch projections around the paged attention kernels.  Slots, positions,
tokens and the step counter advance on the device inside the graph.
"""

from __future__ import annotations

from collections import deque

import torch
import torch.nn.functional as F

from . import ops, paged, step_ops
from .engine import DecodeEngine
from .rope import cos_sin


class PagedDecodeEngine(DecodeEngine):
    """``DecodeEngine`` whose decode step reads and writes a paged KV cache."""

    def new_paged_cache(self, max_rows: int, n_pages: int, page_size: int,
                        pages_per_row: int) -> paged.PagedKvCache:
        cfg = self.cfg
        return paged.PagedKvCache(cfg.layers, cfg.kv_heads, n_pages, page_size, max_rows,
                                  pages_per_row, self.device)

    # ------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill_paged(self, prompts, kv: paged.PagedKvCache, rows):
        """Prompts (list of 1-D id tensors) into rows ``rows`` of ``kv`` (their
        pages mapped beforehand) -> last-token logits (len(rows), vocab).

        One packed varlen launch per layer (``_prefill_ragged`` semantics,
        SE:1162-1204): row b's tokens land in its slots [0, len_b)."""
        rows = list(rows)
        if len(rows) != len(prompts):
            raise ValueError("one row per prompt")
        if rows == list(range(rows[0], rows[0] + len(rows))):
            table = kv.table[rows[0]:rows[0] + len(rows)]
        else:
            table = kv.table[torch.tensor(rows, device=self.device)]
        return self._prefill_packed(
            prompts, lambda i, q, k, v, cu, n, cos, sin, lengths: paged.prefill_varlen_paged(
                q, k, v, cu, n, cos, sin, kv.pools[i][0], kv.pools[i][1], table, 0,
                lengths=lengths))

    # ------------------------------------------------------------------ decode
    def make_paged_context(self, kv: paged.PagedKvCache, batch: int, n_cols: int):
        """Static buffers of the paged graph step over rows [0, batch) of ``kv``.

        ``pos[b]`` is row b's next slot (= its length so far) and its position;
        ``rows[:, step]`` receives each replay's tokens (``n_cols`` columns)."""
        cfg = self.cfg
        dev = self.device
        fused = self.uses_fused_step(batch)
        if fused:
            splits = min(ops.choose_splits(batch, cfg.kv_heads, kv.capacity),
                         self.fused_max_splits(batch))
            flash = ops.make_flash_scratch(batch, cfg.kv_heads, cfg.groups, kv.capacity, dev,
                                           splits=splits, fused=False)
        else:
            flash = ops.make_flash_scratch(batch, cfg.kv_heads, cfg.groups, kv.capacity, dev)
        ctx = {
            "kv": kv,
            "table": kv.table[:batch],
            "flash": flash,
            "token": torch.zeros(batch, device=dev, dtype=torch.long),
            "pos": torch.full((batch,), -1, device=dev, dtype=torch.long),
            "step": torch.zeros(1, device=dev, dtype=torch.long),
            "rows": torch.zeros(batch, n_cols, device=dev, dtype=torch.long),
            "logits": torch.zeros(batch, cfg.vocab, device=dev, dtype=torch.float16),
            "fused": fused,
        }
        if fused:
            f16 = torch.float16
            ctx["hidden"] = torch.zeros(batch, cfg.hidden, device=dev, dtype=f16)
            ctx["q_rot"] = torch.zeros(batch, cfg.heads, cfg.head_dim, device=dev, dtype=f16)
            ctx["h"] = torch.zeros(batch, cfg.intermediate, device=dev, dtype=f16)
            ctx["keys"] = torch.zeros(batch, step_ops.lm_blocks(self.lm_head_weight(batch)),
                                      device=dev, dtype=torch.long)
        return ctx

    def _step(self, ctx):
        if "kv" not in ctx:
            return super()._step(ctx)
        if ctx["fused"]:
            self._step_fused_paged(ctx)
        else:
            self._step_torch_paged(ctx)

    def _step_fused_paged(self, ctx):
        cfg = self.cfg
        b = ctx["token"].shape[0]
        eps = cfg.rms_eps
        kv, table, pos = ctx["kv"], ctx["table"], ctx["pos"]
        rope = (pos, self.inv_freq)                              # each row's own position
        hidden, q_rot, h = ctx["hidden"], ctx["q_rot"], ctx["h"]
        for i, (layer, (kp, vp)) in enumerate(zip(self.w["layers"], kv.pools)):
            w_qkv, w_gate_up = self.projection_weights(i, b)
            if i == 0:
                paged.rms_qkv_rope_append_paged(self.w["embed"], layer["input_norm"], eps,
                                                w_qkv, layer["qkv_bias"], None, None,
                                                kp, vp, table, pos, q_rot, token=ctx["token"],
                                                hidden_out=hidden, positions=rope)
            else:
                paged.rms_qkv_rope_append_paged(hidden, layer["input_norm"], eps,
                                                w_qkv, layer["qkv_bias"], None, None,
                                                kp, vp, table, pos, q_rot, positions=rope)
            grouped = q_rot.view(b, cfg.kv_heads, cfg.groups, cfg.head_dim)
            # The slot just written is the row's last valid one.
            paged.flash_decode_split_paged(grouped, kp, vp, table, None, ctx["flash"], kv_last=pos,
                                           scale=self.scale)
            step_ops.attn_merge_o_proj(ctx["flash"], self.o_proj_weight(i, b), hidden)
            step_ops.rms_gate_up_swiglu(hidden, layer["post_norm"], eps, w_gate_up, h)
            step_ops.gemv_residual(h, layer["down_weight"], hidden)
        step_ops.rms_lm_head(hidden, self.w["final_norm"], eps, self.lm_head_weight(b), ctx["logits"],
                             ctx["keys"])
        step_ops.argmax_step(ctx["keys"], ctx["token"], ctx["rows"], ctx["step"], None, pos)

    def _step_torch_paged(self, ctx):
        cfg = self.cfg
        b = ctx["token"].shape[0]
        kv, table, pos = ctx["kv"], ctx["table"], ctx["pos"]
        hidden = F.embedding(ctx["token"], self.w["embed"]).view(b, 1, cfg.hidden)
        cos, sin = cos_sin(pos, self.inv_freq)
        for layer, (kp, vp) in zip(self.w["layers"], kv.pools):
            residual = hidden
            q, k, v = self._qkv(self._rms(hidden, layer["input_norm"]), layer)
            q_rot = paged.rope_append_paged(q, k, v, cos, sin, kp, vp, table, pos)
            grouped = q_rot.view(b, cfg.kv_heads, cfg.groups, cfg.head_dim)
            att = paged.flash_decode_attention_paged(grouped, kp, vp, table, None, ctx["flash"],
                                                     kv_last=pos, scale=self.scale)
            hidden = residual + F.linear(att.reshape(b, 1, cfg.hidden), layer["o_weight"])
            residual = hidden
            hidden = residual + self._mlp(self._rms(hidden, layer["post_norm"]), layer)
        hidden = self._rms(hidden, self.w["final_norm"]).squeeze(1)
        logits = F.linear(hidden, self.w["lm_head"])
        nxt = torch.argmax(logits, dim=-1)
        ctx["logits"].copy_(logits)
        ctx["token"].copy_(nxt)
        ctx["rows"].index_copy_(1, ctx["step"], nxt.unsqueeze(1))
        pos.add_(1)
        ctx["step"].add_(1)

    def capture_paged(self, ctx):
        """Capture the paged step into a hipGraph.  The two warm-ups run with
        every row parked at slot -1 (nothing is appended, nothing is read); the
        state is restored afterwards."""
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        saved = {k: ctx[k].clone() for k in ("token", "pos", "step", "rows")}
        with torch.cuda.stream(side):
            for _ in range(2):
                ctx["pos"].fill_(-1)
                ctx["step"].fill_(0)
                self._step(ctx)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            self._step(ctx)
        for k, v in saved.items():
            ctx[k].copy_(v)
        torch.cuda.synchronize(self.device)
        ctx["graph"] = graph
        return graph

    # ------------------------------------------------------------------ generation
    @torch.no_grad()
    def generate_paged(self, prompts, max_new_tokens: int, page_size: int = 64,
                       timing: dict | None = None):
        """Greedy ids (B, max_new_tokens) for variable-length prompts, each row
        holding only the pages of its own prompt + new tokens."""
        b = len(prompts)
        lengths = [int(p.numel()) for p in prompts]
        need = [n + max(max_new_tokens - 1, 0) for n in lengths]
        ppr = -(-max(need) // page_size)
        n_pages = sum(-(-n // page_size) for n in need)
        kv = self.new_paged_cache(b, n_pages, page_size, ppr)
        for r, n in enumerate(need):
            kv.map_row(r, n)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record()
        first = torch.argmax(self.prefill_paged(prompts, kv, range(b)), dim=-1)
        ev[1].record()
        ctx = self.make_paged_context(kv, b, max_new_tokens)
        self.capture_paged(ctx)
        ctx["rows"][:, 0] = first
        ctx["token"].copy_(first)
        ctx["pos"].copy_(torch.tensor(lengths, device=self.device))
        ctx["step"].fill_(1)
        torch.cuda.synchronize(self.device)
        ev[2].record()
        for _ in range(1, max_new_tokens):
            ctx["graph"].replay()
        ev[3].record()
        torch.cuda.synchronize(self.device)
        if timing is not None:
            timing["prefill_ms"] = ev[0].elapsed_time(ev[1])
            timing["decode_ms"] = ev[2].elapsed_time(ev[3])
            timing["pages"] = n_pages
        self._ctx = ctx
        return ctx["rows"].clone()

    @torch.no_grad()
    def serve(self, prompts, max_new_tokens, max_batch: int = 4, page_size: int = 64,
              n_pages: int | None = None, stats: dict | None = None):
        """Continuous batching: greedy ids for every prompt (list of 1-D tensors),
        ``max_new_tokens`` an int or one per prompt.

        Up to ``max_batch`` rows decode together in one captured step.  Whenever
        requests finish, their pages return to the pool and the next waiting
        requests (first come, first served) are prefilled, each on its own, into
        the freed rows; the graph then keeps replaying.  A request's tokens do
        not depend on the requests it shares the batch with.  A row with no
        request is parked at slot -1: it appends nothing and its output is
        ignored.  Returns a list of 1-D id tensors, one per prompt.
        """
        n_req = len(prompts)
        news = [max_new_tokens] * n_req if isinstance(max_new_tokens, int) else list(max_new_tokens)
        if len(news) != n_req or min(news) < 1:
            raise ValueError("one max_new_tokens >= 1 per prompt")
        need = [int(p.numel()) + n - 1 for p, n in zip(prompts, news)]
        ppr = -(-max(need) // page_size)
        if n_pages is None:
            n_pages = max_batch * ppr
        kv = self.new_paged_cache(max_batch, n_pages, page_size, ppr)
        # Upper bound on replays: every request decoded back to back.
        ctx = self.make_paged_context(kv, max_batch, sum(n - 1 for n in news) + 1)
        self.capture_paged(ctx)
        ctx["step"].fill_(0)
        queue = deque(range(n_req))
        active = {}                       # row -> (request, first replay, replays left)
        results = [None] * n_req
        replays, admitted = 0, 0

        def admit() -> int:
            """Prefill waiting requests into free rows (again while one-token
            requests free their rows at once); returns how many."""
            total = 0
            while True:
                n = admit_once()
                total += n
                if n == 0 or len(active) == max_batch or not queue:
                    return total

        def admit_once() -> int:
            nonlocal admitted
            free = [r for r in range(max_batch) if r not in active]
            batch = []
            while free and queue and kv.free_pages() >= -(-need[queue[0]] // page_size):
                r, i = free.pop(0), queue.popleft()
                kv.map_row(r, need[i])
                batch.append((r, i))
            if not batch:
                return 0
            rows = [r for r, _ in batch]
            # One prefill per request: its projections then have the same
            # shapes whatever it is admitted with, so its tokens do not depend
            # on the other rows (the decode step is row-independent too).
            first = torch.cat([torch.argmax(self.prefill_paged([prompts[i]], kv, [r]), dim=-1)
                               for r, i in batch])
            idx = torch.tensor(rows, device=self.device)
            ctx["token"].index_copy_(0, idx, first)
            lens = torch.tensor([int(prompts[i].numel()) for _, i in batch], device=self.device)
            ctx["pos"].index_copy_(0, idx, lens)
            for j, (r, i) in enumerate(batch):
                if news[i] == 1:
                    results[i] = first[j:j + 1].clone()
                    kv.release_row(r)
                    ctx["pos"][r] = -1
                else:
                    active[r] = (i, replays, news[i] - 1, first[j:j + 1].clone())
                admitted += 1
            return len(batch)

        admit()
        while active or queue:
            if not active:
                if admit() == 0:
                    raise RuntimeError("page pool too small for the next request")
                continue
            n = min(left for _, _, left, _ in active.values())
            for _ in range(n):
                ctx["graph"].replay()
            replays += n
            for r in list(active):
                i, t0, left, first = active[r]
                if left == n:
                    results[i] = torch.cat([first, ctx["rows"][r, t0:t0 + news[i] - 1]])
                    del active[r]
                    kv.release_row(r)
                    ctx["pos"][r] = -1
                else:
                    active[r] = (i, t0, left - n, first)
            admit()
        torch.cuda.synchronize(self.device)
        if stats is not None:
            stats["replays"] = replays
            stats["requests"] = admitted
            stats["pages"] = n_pages
        self._ctx = ctx
        return results
