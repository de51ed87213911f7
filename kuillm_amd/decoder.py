"""Llama-style decoder on the kuiops kernels: prefill + greedy decode with a
KV cache, the decode step recorded once in a HIP graph and replayed per token.

This is the model the reference runs through ``KuiperMode`` (infer.py:14-31:
a transformers causal LM, bf16, greedy / sampled ``generate``), with every
op of the step on a kuiops kernel:

    embedding        kuiops_index                  (aten.index / embedding)
    RMSNorm (+res)   kuiops_rmsnorm                (pow / mean / rsqrt / mul / add)
    q, k, v          kuiops_decode_linear / mm     one fused [(hq+2hkv) hd, d] weight
    rotary + cache   kuiops_rope_kv_append         (mul / neg / cat / add, cache cat)
    attention        kuiops_sdpa_fwd (prefill), kuiops_sdpa_decode (decode,
                     KV length read from device memory)
    o, gate|up, down kuiops_decode_linear / mm     gate and up fused
    SwiGLU           kuiops_silu_mul (fused into the down projection at decode)
    LM head          kuiops_decode_linear / mm
    sampling tail    kuiops_softmax_lastdim + kuiops_topk_lastdim (k = 1)

Weights stay in the nn.Linear layout [out, in] (q/k/v and gate/up fused
along out).  A batch-1 decode step uses kuiops_decode_linear: every output
is one wave's dot product over a contiguous weight row, with the RMSNorm or
SwiGLU that feeds the projection computed in the same launch.  Prefill
(and batch > 1) uses the MFMA GEMMs on the K-contiguous weights.  Numerics follow the transformers modules (each op
rounds to bf16 where the stock module does), so greedy tokens match the stock
model except where two logits tie within bf16 resolution.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops


@dataclass
class LlamaShape:
    vocab: int
    d: int
    ffn: int
    layers: int
    hq: int
    hkv: int
    eps: float = 1e-5
    theta: float = 10000.0

    @property
    def hd(self) -> int:
        return self.d // self.hq

    @classmethod
    def from_hf(cls, c) -> "LlamaShape":
        theta = getattr(c, "rope_theta", None)
        if theta is None:
            theta = (getattr(c, "rope_parameters", None) or {}).get("rope_theta", 10000.0)
        return cls(vocab=c.vocab_size, d=c.hidden_size, ffn=c.intermediate_size, layers=c.num_hidden_layers,
                   hq=c.num_attention_heads, hkv=c.num_key_value_heads, eps=c.rms_norm_eps, theta=float(theta))


def rope_inv_freq(hd: int, theta: float) -> torch.Tensor:
    """1 / theta^(2i / hd) in fp32, computed as the transformers default rotary init."""
    return 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.int64).float() / hd))


class DecodeStepError(RuntimeError):
    """A persistent decode launch gave up a bounded wait (its work-groups
    were not all resident at once): the tokens of that call are void."""


def persistent_step_ok(s: LlamaShape, batch: int, capacity: int, dtype, fused: bool,
                       supported=None) -> bool:
    """Whether batch-1 decode runs as the persistent step (kuiops_decode_step):
    the fused per-op step must apply, the cache must fit the one-pass
    attention (8 waves x 512 / hd lane groups x 12 keys: the persistent
    attention is the per-op row-wide form, so both give the same bits), and
    the library must accept the shape on this device (its shape gate plus an
    occupancy query that a step work-group fits a CU).  Otherwise decode
    takes the per-op graph."""
    row_wide_keys = 8 * (64 // (s.hd // 8)) * 12
    if not (fused and batch == 1 and s.d == s.hq * s.hd and s.d <= 4096 and s.vocab <= 32768
            and capacity <= row_wide_keys):
        return False
    check = supported if supported is not None else ops.decode_step_supported
    return bool(check(s.layers, s.d, s.ffn, s.hq, s.hkv, s.hd, s.vocab, capacity, dtype))


class LlamaDecoder:
    """Greedy generation for one batch of equal-length prompts.

    ``state`` maps transformers parameter names (``model.layers.{i}.self_attn.q_proj.weight``
    ...) to tensors; ``capacity`` is the KV-cache length (prompt + new tokens).
    """

    def __init__(self, shape: LlamaShape, state: dict, capacity: int, batch: int = 1,
                 device="cuda", dtype=torch.bfloat16):
        self.s = s = shape
        self.cap = int(capacity)
        self.n = int(batch)
        self.dev = torch.device(device)
        self.dtype = dtype
        if s.hd not in (64, 128) or s.hq % s.hkv:
            raise ValueError("head_dim must be 64 or 128 and hq a multiple of hkv")

        def w(name):
            return state[name].to(self.dev, dtype)

        def kn(*names):       # nn.Linear weights [out, in], fused along out: [sum(out), in]
            return torch.cat([w(x) for x in names], 0).contiguous()

        self.embed = w("model.embed_tokens.weight").contiguous()
        self.layers = []
        for i in range(s.layers):
            p = f"model.layers.{i}."
            self.layers.append(dict(
                ln1=w(p + "input_layernorm.weight").contiguous(),
                wqkv=kn(p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight", p + "self_attn.v_proj.weight"),
                wo=kn(p + "self_attn.o_proj.weight"),
                ln2=w(p + "post_attention_layernorm.weight").contiguous(),
                wgu=kn(p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"),
                wd=kn(p + "mlp.down_proj.weight"),
            ))
        self.norm = w("model.norm.weight").contiguous()
        head = state.get("lm_head.weight", state["model.embed_tokens.weight"])
        self.head = head.to(self.dev, dtype).contiguous()
        self.inv_freq = rope_inv_freq(s.hd, s.theta).to(self.dev)
        kv = (s.layers, self.n, s.hkv, self.cap, s.hd)
        self.kcache = torch.zeros(kv, dtype=dtype, device=self.dev)
        self.vcache = torch.zeros(kv, dtype=dtype, device=self.dev)
        # device-side decode state: the token to feed, its position, the key count
        self.tok = torch.zeros(self.n, dtype=torch.int64, device=self.dev)
        # position and key count share one buffer, so a decode step advances
        # both with one launch
        self.step_state = torch.zeros((2, self.n), dtype=torch.int32, device=self.dev)
        self.pos, self.kv_len = self.step_state[0], self.step_state[1]
        self.graph = None
        self.graphs_k = {}
        self.fused = self.n == 1 and s.d <= 4096 and s.ffn <= 8192 and s.d % 8 == 0 and s.ffn % 8 == 0 and s.hd % 2 == 0
        # batches of 2..16: the batched form of the same fused projections
        # (every row of x staged in LDS: n * max(d, ffn) * 2 <= 140 KiB)
        shapes_ok = s.d % 8 == 0 and s.ffn % 8 == 0 and s.hd % 2 == 0
        self.fused_batched = 2 <= self.n <= 16 and self.n * max(s.d, s.ffn) * 2 <= 140 * 1024 and shapes_ok
        # larger batches (up to 64): RMSNorm in its own launch, projections of
        # plain x (read from L2) with the rotary / SwiGLU epilogues fused
        self.fused_wide = not self.fused_batched and 2 <= self.n <= 64 and shapes_ok
        # batch 1: the whole step as one persistent launch
        # (kuiops_decode_step) when its attention has the one-pass row-wide
        # form of the per-op path (the cache fits 8 waves x 12 keys per lane
        # group), so both paths give the same bits
        self.persistent = persistent_step_ok(s, self.n, self.cap, dtype, self.fused)
        # persistent launches run up to this many steps each (the next step's
        # weights stream while a step's LM head and sampling run); decode()
        # covers a token count with launches of 32, 16, 8, 4, 2 and 1 steps
        self.steps_per_launch = 32 if self.persistent else 1
        if self.fused or self.fused_batched or self.fused_wide:
            self._setup_fused()

    def _setup_fused(self):
        """Static buffers of the batch-1 decode step, whose projections carry
        their input stage (RMSNorm) and epilogue (rotary + KV append, SwiGLU):
        5 launches per layer."""
        s, dev, n = self.s, self.dev, self.n
        bf = dict(dtype=self.dtype, device=dev)
        if n == 1:
            self.h_buf = [torch.empty(s.d, **bf), torch.empty(s.d, **bf)]
            self.q1 = torch.empty(1, s.hq, 1, s.hd, **bf)
            self.att1 = torch.empty(1, 1, s.hq * s.hd, **bf)
            self.o1 = torch.empty(s.d, **bf)
            self.a1 = torch.empty(s.ffn, **bf)
            self.down1 = torch.empty(s.d, **bf)
            self.logits1 = torch.empty(s.vocab, **bf)
        else:
            self.h_buf = [torch.empty(n, s.d, **bf), torch.empty(n, s.d, **bf)]
            self.qb = torch.empty(n, s.hq * s.hd, **bf)
            self.attb = torch.empty(n, s.hq * s.hd, **bf)
            self.ob = torch.empty(n, s.d, **bf)
            self.ab = torch.empty(n, s.ffn, **bf)
            self.downb = torch.empty(n, s.d, **bf)
            self.logitsb = torch.empty(n, s.vocab, **bf)
            self.xnb = torch.empty(n, s.d, **bf)          # wide step: normalised rows
        self.top_v = torch.empty(n, 1, dtype=torch.float32, device=dev)
        if self.persistent:
            ptrs = [[L[k].data_ptr() for k in ("wqkv", "wo", "wgu", "wd", "ln1", "ln2")]
                    + [self.kcache[i, 0].data_ptr(), self.vcache[i, 0].data_ptr()]
                    for i, L in enumerate(self.layers)]
            self.layer_table = torch.tensor(ptrs, dtype=torch.int64, device=dev)
            self.step_sync = torch.zeros(ops.decode_step_sync_bytes(s.layers), dtype=torch.uint8, device=dev)
            self.step_scratch = torch.zeros(
                ops.decode_step_scratch_bytes(s.layers, self.steps_per_launch, s.d, s.ffn, s.hq, s.hkv, s.hd),
                dtype=torch.uint8, device=dev)
        # token chosen at each position (written by the step itself, so a
        # replayed step needs no copy out)
        self.history = torch.zeros(n, self.cap + 1, dtype=torch.int64, device=dev)

    @classmethod
    def from_hf(cls, model, capacity: int, batch: int = 1, device="cuda"):
        return cls(LlamaShape.from_hf(model.config), model.state_dict(), capacity, batch, device)

    # ------------------------------------------------------------ forward

    def _layers(self, h, t, pos0, kv_len):
        """Run every layer on h [n * t, d] (t new tokens per sequence at
        positions pos0 ..); returns the final-norm input (last MLP output)
        and the residual stream."""
        s, n = self.s, self.n
        res = h
        pending = None
        q = torch.empty((n, s.hq, t, s.hd), dtype=self.dtype, device=self.dev)
        att = torch.empty((n, t, s.hq * s.hd), dtype=self.dtype, device=self.dev)
        att4 = att.view(n, t, s.hq, s.hd).transpose(1, 2)            # [n, hq, t, hd] view
        for i, L in enumerate(self.layers):
            if pending is None:
                x = ops.rmsnorm(res, L["ln1"], s.eps)
            else:
                x = ops.rmsnorm(pending, L["ln1"], s.eps, residual=res, res_out=res)
            qkv = ops.mm(x, L["wqkv"].t()).view(n, t, -1)
            kc, vc = self.kcache[i], self.vcache[i]
            ops.rope_kv_append(qkv, s.hq, s.hkv, s.hd, self.inv_freq, pos0, q, kc, vc)
            if t == 1:
                ops.sdpa_decode(q, kc, vc, causal=True, kv_len=kv_len, out=att4)
            else:
                # prefill from position 0: the keys are the t just stored
                ops.sdpa(q, kc[:, :, :t], vc[:, :, :t], is_causal=True, return_lse=False, out=att4)
            o = ops.mm(att.view(n * t, -1), L["wo"].t())
            x = ops.rmsnorm(o, L["ln2"], s.eps, residual=res, res_out=res)
            a = ops.silu_mul(ops.mm(x, L["wgu"].t()))
            pending = ops.mm(a, L["wd"].t())
        return pending, res

    def _head(self, pending, res, t):
        """Greedy next token of each sequence from its last position."""
        n = self.n
        last = (lambda z: z.view(n, t, -1)[:, -1]) if t > 1 else (lambda z: z)
        x = ops.rmsnorm(last(pending), self.norm, self.s.eps, residual=last(res))
        logits = ops.mm(x, self.head.t())                           # bf16, as the stock LM head
        probs = ops.softmax(logits.float())
        _, idx = ops.topk(probs, 1)
        return logits, idx.view(n)

    def prefill(self, prompt: torch.Tensor):
        """Run the prompt [n, t] (positions 0 .. t-1) and fill the KV cache;
        returns (last-position logits [n, vocab], next tokens [n])."""
        n, t = prompt.shape
        if n != self.n or t > self.cap:
            raise ValueError("prompt does not fit the batch / cache")
        ids = prompt.to(self.dev).reshape(-1).contiguous()
        h = ops.index(self.embed, 0, ids)
        self.pos.zero_()
        pending, res = self._layers(h, t, self.pos, None)
        logits, nxt = self._head(pending, res, t)
        self.tok.copy_(nxt)
        self.pos.fill_(t)
        self.kv_len.fill_(t + 1)
        return logits, nxt

    def _decode_step(self, n_steps: int = 1):
        if n_steps != 1 and not self.persistent:
            raise ValueError("several steps per launch need the persistent step")
        if self.fused:
            return self._decode_step_fused(n_steps)
        if self.fused_batched:
            return self._decode_step_fused_batched()
        if self.fused_wide:
            return self._decode_step_wide()
        h = ops.index(self.embed, 0, self.tok)
        pending, res = self._layers(h, 1, self.pos, self.kv_len)
        logits, nxt = self._head(pending, res, 1)
        self.tok.copy_(nxt)
        self.step_state.add_(1)
        return logits

    def _decode_step_fused(self, n_steps: int = 1):
        """One batch-1 decode step, same arithmetic as ``_layers`` + ``_head``
        (every rounding point kept), in 5 launches per layer plus LM head and
        a fused softmax / top-1 / state-advance launch: qkv (embedding
        lookup / RMSNorm stage, rotary + cache append epilogue) -> attention
        -> o -> gate|up (RMSNorm stage, SwiGLU epilogue) -> down.  With
        ``persistent`` the same work, bit for bit, runs as one launch, which
        can also run ``n_steps`` consecutive steps."""
        s = self.s
        if self.persistent:
            ops.decode_step(self.layer_table, s.layers, s.d, s.ffn, s.hq, s.hkv, s.hd, s.vocab, s.eps,
                            self.kcache[0, 0], self.vcache[0, 0], self.embed, self.norm, self.head, self.inv_freq,
                            self.tok, self.pos, self.kv_len, self.history[0], self.top_v.view(1),
                            self.logits1, self.step_scratch, self.step_sync, n_steps=n_steps)
            return self.logits1.view(1, -1)
        hb = self.h_buf
        cur = 0
        att4 = self.att1.view(1, 1, s.hq, s.hd).transpose(1, 2)
        down = None
        for i, L in enumerate(self.layers):
            kc, vc = self.kcache[i], self.vcache[i]
            src = self.embed if i == 0 else hb[cur]
            ops.decode_qkv_rope(src, L["wqkv"], s.hq, s.hkv, s.hd, self.inv_freq, self.pos, self.q1, kc[0], vc[0],
                                x_kind="rmsnorm", row=self.tok if i == 0 else None, in_add=down,
                                norm_w=L["ln1"], eps=s.eps, h_out=hb[1 - cur])
            cur = 1 - cur
            ops.sdpa_decode(self.q1, kc, vc, causal=True, kv_len=self.kv_len, out=att4)
            ops.decode_linear(self.att1, L["wo"], "plain", out=self.o1)
            ops.decode_gate_up(hb[cur], L["wgu"], "rmsnorm", in_add=self.o1, norm_w=L["ln2"], eps=s.eps,
                               h_out=hb[1 - cur], out=self.a1)
            cur = 1 - cur
            ops.decode_linear(self.a1, L["wd"], "plain", out=self.down1)
            down = self.down1
        ops.decode_linear(hb[cur], self.head, "rmsnorm", in_add=down, norm_w=self.norm, eps=s.eps,
                          out=self.logits1)
        # softmax(logits.float()) + top-1 and the position / key-count
        # advance, in one launch (same probabilities and order as the
        # softmax + topk pair of _head)
        ops.softmax_top1(self.logits1.view(1, -1), index_out=self.tok, prob_out=self.top_v.view(1),
                         pos=self.pos, kv_len=self.kv_len, history=self.history)
        return self.logits1.view(1, -1)

    def _decode_step_fused_batched(self):
        """One decode step for a batch of 2..16 sequences with the batched
        fused projections (kuiops_decode_rows_batched): the same 5 launches per
        layer as the batch-1 step, each sequence at its own position."""
        s, n = self.s, self.n
        hb = self.h_buf
        cur = 0
        q4 = self.qb.view(n, s.hq, 1, s.hd)
        att4 = self.attb.view(n, s.hq, 1, s.hd)
        down = None
        for i, L in enumerate(self.layers):
            kc, vc = self.kcache[i], self.vcache[i]
            src = self.embed if i == 0 else hb[cur]
            ops.decode_rows_batched(src, L["wqkv"], "rmsnorm", "rope", in_add=down, norm_w=L["ln1"], eps=s.eps,
                                    h_out=hb[1 - cur], out=self.qb, row=self.tok if i == 0 else None,
                                    hq=s.hq, hkv=s.hkv, hd=s.hd, inv_freq=self.inv_freq, pos=self.pos,
                                    k_cache=kc, v_cache=vc)
            cur = 1 - cur
            ops.sdpa_decode(q4, kc, vc, causal=True, kv_len=self.kv_len, out=att4)
            ops.decode_rows_batched(self.attb, L["wo"], "plain", "plain", out=self.ob)
            ops.decode_rows_batched(hb[cur], L["wgu"], "rmsnorm", "swiglu", in_add=self.ob, norm_w=L["ln2"],
                                    eps=s.eps, h_out=hb[1 - cur], out=self.ab)
            cur = 1 - cur
            ops.decode_rows_batched(self.ab, L["wd"], "plain", "plain", out=self.downb)
            down = self.downb
        ops.decode_rows_batched(hb[cur], self.head, "rmsnorm", "plain", in_add=down, norm_w=self.norm, eps=s.eps,
                                out=self.logitsb)
        ops.softmax_top1(self.logitsb, index_out=self.tok, prob_out=self.top_v.view(n),
                         pos=self.pos, kv_len=self.kv_len, history=self.history)
        return self.logitsb

    def _decode_step_wide(self):
        """One decode step for a batch of up to 64 sequences: the unfused
        step's arithmetic with the projections on kuiops_decode_rows_batched
        (plain x; rotary + KV append and SwiGLU in their epilogues), 7
        launches per layer."""
        s, n = self.s, self.n
        res, xn = self.h_buf[0], self.xnb
        q4 = self.qb.view(n, s.hq, 1, s.hd)
        att4 = self.attb.view(n, s.hq, 1, s.hd)
        ops.index(self.embed, 0, self.tok, out=res)
        for i, L in enumerate(self.layers):
            kc, vc = self.kcache[i], self.vcache[i]
            if i == 0:
                ops.rmsnorm(res, L["ln1"], s.eps, out=xn)
            else:
                ops.rmsnorm(self.downb, L["ln1"], s.eps, residual=res, res_out=res, out=xn)
            ops.decode_rows_batched(xn, L["wqkv"], "plain", "rope", out=self.qb, hq=s.hq, hkv=s.hkv, hd=s.hd,
                                    inv_freq=self.inv_freq, pos=self.pos, k_cache=kc, v_cache=vc)
            ops.sdpa_decode(q4, kc, vc, causal=True, kv_len=self.kv_len, out=att4)
            ops.decode_rows_batched(self.attb, L["wo"], "plain", "plain", out=self.ob)
            ops.rmsnorm(self.ob, L["ln2"], s.eps, residual=res, res_out=res, out=xn)
            ops.decode_rows_batched(xn, L["wgu"], "plain", "swiglu", out=self.ab)
            ops.decode_rows_batched(self.ab, L["wd"], "plain", "plain", out=self.downb)
        ops.rmsnorm(self.downb, self.norm, s.eps, residual=res, out=xn)
        ops.decode_rows_batched(xn, self.head, "plain", "plain", out=self.logitsb)
        ops.softmax_top1(self.logitsb, index_out=self.tok, prob_out=self.top_v.view(n),
                         pos=self.pos, kv_len=self.kv_len, history=self.history)
        return self.logitsb

    def capture(self):
        """Record one decode step (all its kernels) in a HIP graph, and with
        the persistent step also one launch of steps_per_launch steps.  The
        step reads the token, position and key count from device memory and
        advances them, so replays need no host work."""
        saved = (self.tok.clone(), self.pos.clone(), self.kv_len.clone(),
                 self.kcache.clone(), self.vcache.clone())

        def record(n_steps):
            self._decode_step(n_steps)                   # eager: allocates workspaces
            torch.cuda.synchronize(self.dev)
            g = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream(self.dev)
            side.wait_stream(torch.cuda.current_stream(self.dev))
            with torch.cuda.stream(side):
                self._decode_step(n_steps)
            torch.cuda.current_stream(self.dev).wait_stream(side)
            with torch.cuda.graph(g):
                logits = self._decode_step(n_steps)
            torch.cuda.synchronize(self.dev)
            for dst, src in zip((self.tok, self.pos, self.kv_len, self.kcache, self.vcache), saved):
                dst.copy_(src)
            return g, logits

        # graphs of 2, 4, ... steps_per_launch steps (the capacity must hold
        # the steps the recording runs)
        self.graphs_k = {}
        if self.persistent:
            k = 2
            while k <= self.steps_per_launch and int(self.pos[0]) + 3 * k <= self.cap:
                self.graphs_k[k], _ = record(k)
                k *= 2
        self.graph, self.graph_logits = record(1)

    def decode(self, n_new: int, use_graph: bool = True) -> torch.Tensor:
        """Greedy-decode n_new tokens after ``prefill``; returns [n, n_new]
        (the first is the token prefill chose)."""
        out = torch.empty((n_new, self.n), dtype=torch.int64, device=self.dev)
        if n_new == 0:
            return out.t()
        if int(self.pos[0]) + n_new - 1 > self.cap:
            raise ValueError("KV cache too small")
        if use_graph and self.graph is None:
            self.capture()
        out[0].copy_(self.tok)
        p0 = int(self.pos[0])
        i = 1
        while i < n_new:
            # the largest multi-step launch that fits the tokens left
            k = self.steps_per_launch if self.persistent else 1
            while k > 1 and (k > n_new - i or (use_graph and k not in self.graphs_k)):
                k //= 2
            if k > 1:
                if use_graph:
                    self.graphs_k[k].replay()
                else:
                    self._decode_step(k)
                i += k
                continue
            if use_graph:
                self.graph.replay()
            else:
                self._decode_step()
            if not (self.fused or self.fused_batched or self.fused_wide):
                out[i].copy_(self.tok)
            i += 1
        if self.persistent:
            self.check_step_error()
        if (self.fused or self.fused_batched or self.fused_wide) and n_new > 1:
            # the fused step recorded the token of position p at history[p]
            out[1:].copy_(self.history[:, p0:p0 + n_new - 1].t())
        return out.t()

    def check_step_error(self):
        """Raises DecodeStepError when a persistent launch on this decoder
        gave up a bounded wait (one 4-byte read, synchronising the stream;
        the flag is cleared, and launches do no work while it is set)."""
        if ops.decode_step_error(self.step_sync, self.s.layers):
            raise DecodeStepError("persistent decode step: a cross-work-group wait expired "
                                  "(work-groups not co-resident); the decoded tokens are void")

    def generate(self, prompt: torch.Tensor, n_new: int, use_graph: bool = True) -> torch.Tensor:
        self.prefill(prompt)
        return self.decode(n_new, use_graph)
