"""A random-init Llama-shaped decoder built only from torch.ops.fxpr.* (test
harness): embedding -> [RMSNorm -> merged q/k/v GEMM -> RoPE -> KV-cache
write -> paged attention -> o GEMM -> residual RMSNorm -> merged gate/up GEMM
-> SiLU * up -> down GEMM] x L -> final RMSNorm -> lm_head GEMM (each
request's last token) ->
greedy sampler with top-k log-probabilities (sample_greedy_fxp), plus the full
fixed-point log-probability row (log_softmax_fxp) when asked.

Every reduction runs in a fixed-point kernel; the rest (embedding lookup,
RoPE, SiLU, products) is elementwise, so a request's tokens and
log-probabilities must not depend on which other requests share its batch or
whether they are prefilling or decoding. The continuous-batching scheduler
here runs any mix of prefills and decodes in one flat token batch, like
vLLM's. Config() is a small model; Config.llama3_8b() is BASELINE config 5's
shape (32 layers, hidden 4096, 32 / 8 heads of 128, FFN 14336, vocab 128256).
The q/k/v and gate/up projections are one weight each ([(Hq + 2 Hkv) D, hidden]
and [2 FFN, hidden]), as vLLM's QKVParallelLinear and MergedColumnParallelLinear
hold them, so a layer runs four GEMMs (N = 6144, 4096, 28672, 4096 at the
Llama-3-8B shape). Weights are drawn on the device from a seeded generator.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

import torch


@dataclass
class Config:
    vocab: int = 1024
    hidden: int = 256
    layers: int = 2
    heads: int = 4
    kv_heads: int = 2
    head_dim: int = 64
    ffn: int = 512
    page: int = 16
    pages: int = 512
    eps: float = 1e-6
    int_bits: int = 32
    frac_bits: int = 16
    dtype: torch.dtype = torch.bfloat16
    num_logprobs: int = 5          # top-k log-probabilities per sampled token
    full_logprobs: bool = True     # also keep the whole log-probability row

    @classmethod
    def llama3_8b(cls, pages: int) -> "Config":
        return replace(cls(), vocab=128_256, hidden=4096, layers=32, heads=32, kv_heads=8, head_dim=128,
                       ffn=14_336, pages=pages, full_logprobs=False)


class Decoder:
    def __init__(self, cfg: Config, seed: int = 0, device: str = "cuda"):
        self.cfg, self.dev = cfg, device
        g = torch.Generator(device).manual_seed(seed)
        c, d = cfg, cfg.dtype

        def w(*shape, std=0.02, mean=0.0):
            return (torch.randn(*shape, generator=g, device=device) * std + mean).to(d)

        self.embed = w(c.vocab, c.hidden, std=1.0)
        self.layers = []
        for _ in range(c.layers):
            self.layers.append({
                "ln1": w(c.hidden, std=0.1, mean=1.0),
                "wqkv": w((c.heads + 2 * c.kv_heads) * c.head_dim, c.hidden),
                "wo": w(c.hidden, c.heads * c.head_dim),
                "ln2": w(c.hidden, std=0.1, mean=1.0),
                "wgu": w(2 * c.ffn, c.hidden), "wd": w(c.hidden, c.ffn),
            })
        self.ln_f = w(c.hidden, std=0.1, mean=1.0)
        self.lm_head = w(c.vocab, c.hidden)
        # one KV cache per layer; pages handed out per request
        self.kv = [torch.zeros(c.pages, 2, c.page, c.kv_heads, c.head_dim, dtype=d, device=device)
                   for _ in range(c.layers)]
        inv = 1.0 / (10000.0 ** (torch.arange(0, c.head_dim, 2, dtype=torch.float32) / c.head_dim))
        self.inv_freq = inv.to(device)

    def reset_cache(self):
        for kv in self.kv:
            kv.zero_()

    def _gemm(self, x, w):  # x [T, K], w [N, K] (vLLM layout) -> [T, N]
        c = self.cfg
        return torch.ops.fxpr.gemm_fxp(x, w.t(), None, c.int_bits, c.frac_bits)

    def _rope_tables(self, pos):  # once per step: [T, 1, D] cos and signed sin
        ang = pos.to(torch.float32)[:, None] * self.inv_freq[None, :]
        cos, sin = torch.cos(ang), torch.sin(ang)
        return torch.cat([cos, cos], -1)[:, None, :], torch.cat([-sin, sin], -1)[:, None, :]

    def _rope(self, x, tables):  # x [T, H, D], rotate-half, fp32 math per element
        # x1 cos - x2 sin | x2 cos + x1 sin: each product rounded, then one
        # add (x2 * -sin is exactly -(x2 * sin)); q and k heads in one call
        # (x is widened to fp32 inside each product: the same values as
        # converting it first, one kernel fewer)
        cos, sin = tables
        T, H, D = x.shape
        out = x * cos
        out += x.view(T, H, 2, D // 2).flip(2).reshape(T, H, D) * sin
        return out.to(x.dtype)

    def step(self, tokens, positions, qsl, seq_lens, block_table, slots, max_q, sample_rows):
        """One forward over a flat batch. Returns, for the token rows
        `sample_rows`: (token ids, their log-probs, top-k ids, top-k log-probs,
        full log-prob rows or None)."""
        c = self.cfg
        T = tokens.shape[0]
        h = self.embed[tokens]
        residual = None
        rope = self._rope_tables(positions)
        for li, L in enumerate(self.layers):
            if residual is None:
                residual = h.clone()
                x = torch.ops.fxpr.rms_norm_fxp(h, L["ln1"], c.eps)
            else:
                x = torch.ops.fxpr.rms_norm_fxp_residual(h, residual, L["ln1"], c.eps)
            qkv = self._gemm(x, L["wqkv"])
            nq, nkv = c.heads * c.head_dim, c.kv_heads * c.head_dim
            qk = self._rope(qkv[:, :nq + nkv].view(T, c.heads + c.kv_heads, c.head_dim), rope)
            q, k = qk[:, :c.heads], qk[:, c.heads:]
            v = qkv[:, nq + nkv:].view(T, c.kv_heads, c.head_dim)
            torch.ops.fxpr.reshape_and_cache(k, v, self.kv[li], slots)
            o = torch.empty(T, c.heads, c.head_dim, dtype=q.dtype, device=q.device)
            torch.ops.fxpr.unified_attention_fxp(q, self.kv[li], o, qsl, seq_lens, block_table, max_q, None,
                                                 True, c.head_dim ** -0.5, c.int_bits, c.frac_bits, 0.0, 0, 0)
            del q, k, v, qk, qkv
            h = self._gemm(o.view(T, -1), L["wo"])
            x = torch.ops.fxpr.rms_norm_fxp_residual(h, residual, L["ln2"], c.eps)
            gu = self._gemm(x, L["wgu"])
            # (both halves widened by one copy: an in-place product with the
            # bf16 half itself takes a slow path at one row, ~48 us)
            guf = gu.float()
            act = torch.nn.functional.silu(guf[:, :c.ffn])
            act.mul_(guf[:, c.ffn:])
            h = self._gemm(act.to(c.dtype), L["wd"])
            del act, gu, guf
        x = torch.ops.fxpr.rms_norm_fxp_residual(h, residual, self.ln_f, c.eps)
        logits = self._gemm(x[sample_rows].contiguous(), self.lm_head)
        ids, lp, top, top_lp = torch.ops.fxpr.sample_greedy_fxp(logits, c.num_logprobs, c.int_bits, c.frac_bits)
        full = (torch.ops.fxpr.log_softmax_fxp(logits, c.int_bits, c.frac_bits, torch.float32)
                if c.full_logprobs else None)
        return ids, lp, top, top_lp, full


TinyDecoder = Decoder


@dataclass
class Request:
    rid: int
    prompt: list[int]
    max_new: int
    pages: list[int] = field(default_factory=list)
    tokens: list[int] = field(default_factory=list)   # prompt + generated
    cached: int = 0                                   # tokens already in the KV cache
    logprobs: list[torch.Tensor] = field(default_factory=list)   # per step: the sampled token's
    topk: list[tuple[torch.Tensor, torch.Tensor]] = field(default_factory=list)
    full: list[torch.Tensor] = field(default_factory=list)

    @property
    def done(self):
        return len(self.tokens) - len(self.prompt) >= self.max_new


def run(model: Decoder, prompts: list[list[int]], max_new: int, schedule) -> dict[int, Request]:
    """Greedy generation. ``schedule(step, active) -> list of requests`` picks
    which unfinished requests run in each forward (a prefill runs the whole
    uncached prompt, a decode one token)."""
    c = model.cfg
    model.reset_cache()
    reqs = {i: Request(i, p, max_new, tokens=list(p)) for i, p in enumerate(prompts)}
    free = list(range(c.pages))
    max_pages = -(-max(len(p) + max_new for p in prompts) // c.page)
    step = 0
    while any(not r.done for r in reqs.values()):
        batch = schedule(step, [r for r in reqs.values() if not r.done])
        step += 1
        if not batch:
            continue
        toks, pos, slots, qsl, sls, bts = [], [], [], [0], [], []
        for r in batch:
            new = r.tokens[r.cached:]
            need = -(-len(r.tokens) // c.page)
            while len(r.pages) < need:
                r.pages.append(free.pop(0))
            for j, t in enumerate(new):
                p = r.cached + j
                toks.append(t)
                pos.append(p)
                slots.append(r.pages[p // c.page] * c.page + p % c.page)
            qsl.append(qsl[-1] + len(new))
            sls.append(len(r.tokens))
            bts.append(r.pages + [0] * (max_pages - len(r.pages)))
        dev = model.dev
        last = [qsl[i + 1] - 1 for i in range(len(batch))]
        ids, lp, top, top_lp, full = model.step(
            torch.tensor(toks, device=dev), torch.tensor(pos, device=dev),
            torch.tensor(qsl, dtype=torch.int32, device=dev), torch.tensor(sls, dtype=torch.int32, device=dev),
            torch.tensor(bts, dtype=torch.int32, device=dev), torch.tensor(slots, dtype=torch.int64, device=dev),
            max(qsl[i + 1] - qsl[i] for i in range(len(batch))), torch.tensor(last, device=dev))
        ids, lp, top, top_lp = ids.cpu(), lp.cpu(), top.cpu(), top_lp.cpu()
        full = None if full is None else full.cpu()
        for i, r in enumerate(batch):
            r.logprobs.append(lp[i])
            r.topk.append((top[i], top_lp[i]))
            if full is not None:
                r.full.append(full[i])
            r.cached = len(r.tokens)
            r.tokens.append(int(ids[i]))
    return reqs


def run_graph(model: Decoder, prompts: list[list[int]], max_new: int, timing: dict | None = None) -> dict[int, Request]:
    """Greedy generation as a serving loop runs it: every prompt prefilled in
    one flat eager step, one eager decode step (which also settles the
    allocator and first-launch set-up), then the remaining decode steps
    replayed from one captured HIP graph, as vLLM serves decode batches. A
    replay decodes one token for every request and advances the decode state
    on the device (next token, position, context length, cache slot), so the
    replays queue back to back with no host synchronisation. Each request
    gets the pages for its prompt and all its new tokens up front. Returns
    the requests as run() does (the bits must match it: no op's result depends
    on page placement or on graph replay). If `timing` is a dict it receives
    `prefill_s`, and `decode_s` / `decode_steps` for the replayed steps
    (device-synchronised wall time)."""
    import time

    c, dev = model.cfg, model.dev
    model.reset_cache()
    B = len(prompts)
    reqs = {i: Request(i, p, max_new, tokens=list(p)) for i, p in enumerate(prompts)}
    max_pages = -(-max(len(p) + max_new for p in prompts) // c.page)
    nxt = 0
    for r in reqs.values():
        need = -(-(len(r.prompt) + max_new) // c.page)
        r.pages = list(range(nxt, nxt + need))
        nxt += need
    if nxt > c.pages:
        raise ValueError(f"run_graph: {nxt} pages needed, the cache holds {c.pages}")
    toks, pos, slots, qsl = [], [], [], [0]
    for r in reqs.values():
        for p, t in enumerate(r.prompt):
            toks.append(t)
            pos.append(p)
            slots.append(r.pages[p // c.page] * c.page + p % c.page)
        qsl.append(qsl[-1] + len(r.prompt))
    bt = torch.tensor([r.pages + [0] * (max_pages - len(r.pages)) for r in reqs.values()],
                      dtype=torch.int32, device=dev)
    plen = torch.tensor([len(r.prompt) for r in reqs.values()], dtype=torch.int32, device=dev)
    hist = []   # per step: (ids, log-prob, top-k ids, top-k log-probs, full row or None), on the device

    def keep(out):
        hist.append(tuple(None if o is None else o.clone() for o in out))

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = model.step(torch.tensor(toks, device=dev), torch.tensor(pos, device=dev),
                     torch.tensor(qsl, dtype=torch.int32, device=dev), plen, bt,
                     torch.tensor(slots, dtype=torch.int64, device=dev), max(len(p) for p in prompts),
                     torch.tensor(qsl[1:], device=dev) - 1)
    keep(out)
    torch.cuda.synchronize()
    if timing is not None:
        timing["prefill_s"] = time.perf_counter() - t0

    tok_d = out[0].clone()
    pos_d = plen.to(torch.int64)          # position of the token fed in
    sl_d = plen + 1                       # context length including it
    slot_d = torch.empty(B, dtype=torch.int64, device=dev)
    qsl_d = torch.arange(B + 1, dtype=torch.int32, device=dev)
    rows = torch.arange(B, device=dev)

    def body():
        slot_d.copy_(bt[rows, pos_d // c.page].to(torch.int64) * c.page + pos_d % c.page)
        o = model.step(tok_d, pos_d, qsl_d, sl_d, bt, slot_d, 1, rows)
        tok_d.copy_(o[0])
        pos_d.add_(1)
        sl_d.add_(1)
        return o

    if max_new >= 2:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):      # the first decode step, eager
            keep(body())
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
    if max_new >= 3:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            gout = body()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(max_new - 2):
            graph.replay()
            keep(gout)
        torch.cuda.synchronize()
        if timing is not None:
            timing["decode_s"] = time.perf_counter() - t0
            timing["decode_steps"] = max_new - 2
        del graph, gout
    for s, (ids, lp, top, top_lp, full) in enumerate(hist):
        ids, lp, top, top_lp = ids.cpu(), lp.cpu(), top.cpu(), top_lp.cpu()
        full = None if full is None else full.cpu()
        for i, r in enumerate(reqs.values()):
            r.logprobs.append(lp[i])
            r.topk.append((top[i], top_lp[i]))
            if full is not None:
                r.full.append(full[i])
            r.tokens.append(int(ids[i]))
    for r in reqs.values():
        r.cached = len(r.tokens) - 1
    return reqs
