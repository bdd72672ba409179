"""A random-init Llama-shaped decoder built only from torch.ops.fxpr.* (test
harness): embedding -> [RMSNorm -> q/k/v GEMMs -> RoPE -> KV-cache write ->
paged attention -> o GEMM -> residual RMSNorm -> gate/up GEMMs -> SiLU * up ->
down GEMM] x L -> final RMSNorm -> lm_head GEMM (each request's last token) ->
greedy sampler with top-k log-probabilities (sample_greedy_fxp), plus the full
fixed-point log-probability row (log_softmax_fxp) when asked.

Every reduction runs in a fixed-point kernel; the rest (embedding lookup,
RoPE, SiLU, products) is elementwise, so a request's tokens and
log-probabilities must not depend on which other requests share its batch or
whether they are prefilling or decoding. The continuous-batching scheduler
here runs any mix of prefills and decodes in one flat token batch, like
vLLM's. Config() is a small model; Config.llama3_8b() is BASELINE config 5's
shape (32 layers, hidden 4096, 32 / 8 heads of 128, FFN 14336, vocab 128256).
Weights are drawn on the device from a seeded generator.
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
                "wq": w(c.heads * c.head_dim, c.hidden), "wk": w(c.kv_heads * c.head_dim, c.hidden),
                "wv": w(c.kv_heads * c.head_dim, c.hidden), "wo": w(c.hidden, c.heads * c.head_dim),
                "ln2": w(c.hidden, std=0.1, mean=1.0),
                "wg": w(c.ffn, c.hidden), "wu": w(c.ffn, c.hidden), "wd": w(c.hidden, c.ffn),
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

    def _rope(self, x, pos):  # x [T, H, D], rotate-half, fp32 math per element
        ang = pos.to(torch.float32)[:, None] * self.inv_freq[None, :]
        cos, sin = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
        xf = x.float()
        x1, x2 = xf[..., : x.shape[-1] // 2], xf[..., x.shape[-1] // 2:]
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)

    def step(self, tokens, positions, qsl, seq_lens, block_table, slots, max_q, sample_rows):
        """One forward over a flat batch. Returns, for the token rows
        `sample_rows`: (token ids, their log-probs, top-k ids, top-k log-probs,
        full log-prob rows or None)."""
        c = self.cfg
        T = tokens.shape[0]
        h = self.embed[tokens]
        residual = None
        for li, L in enumerate(self.layers):
            if residual is None:
                residual = h.clone()
                x = torch.ops.fxpr.rms_norm_fxp(h, L["ln1"], c.eps)
            else:
                x = torch.ops.fxpr.rms_norm_fxp_residual(h, residual, L["ln1"], c.eps)
            q = self._rope(self._gemm(x, L["wq"]).view(T, c.heads, c.head_dim), positions)
            k = self._rope(self._gemm(x, L["wk"]).view(T, c.kv_heads, c.head_dim), positions)
            v = self._gemm(x, L["wv"]).view(T, c.kv_heads, c.head_dim)
            torch.ops.fxpr.reshape_and_cache(k, v, self.kv[li], slots)
            o = torch.empty_like(q)
            torch.ops.fxpr.unified_attention_fxp(q, self.kv[li], o, qsl, seq_lens, block_table, max_q, None,
                                                 True, c.head_dim ** -0.5, c.int_bits, c.frac_bits, 0.0, 0, 0)
            del q, k, v
            h = self._gemm(o.view(T, -1), L["wo"])
            x = torch.ops.fxpr.rms_norm_fxp_residual(h, residual, L["ln2"], c.eps)
            act = torch.nn.functional.silu(self._gemm(x, L["wg"]).float())
            act.mul_(self._gemm(x, L["wu"]).float())
            h = self._gemm(act.to(c.dtype), L["wd"])
            del act
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
