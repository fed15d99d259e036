"""fp32 PyTorch-CPU restatement of the reference's decoder and its
speculative loop (oracle side; also the timed CPU baseline).

Follows nano_sglang/model/causal_lm.py:
  * ModelConfig fields and head_dim = hidden / heads (causal_lm.py:77-101);
  * RMSNorm fallback: variance in fp32, ``x * rsqrt(var + eps)``, then
    ``weight * x`` cast back (causal_lm.py:139-145); fused residual variant
    ``residual = residual + x; return norm(residual), residual``
    (causal_lm.py:147-154);
  * RoPE tables ``theta ** (arange(0, D, 2) / D)`` in fp32 (causal_lm.py:
    157-164) and the half-split rotation with cos/sin cast to x's dtype before
    the multiply (causal_lm.py:167-206);
  * Attention.forward on a contiguous cache: write cache[:, :, pos:pos+S],
    read [:, :, :pos+S], repeat_interleave for GQA, scores / sqrt(D) + mask,
    softmax in fp32, P @ V, o_proj (causal_lm.py:224-262);
  * DecoderLayer / SwiGLU MLP / CausalLM.forward (causal_lm.py:474-583).

And nano_sglang/decode/speculative.py:50-184 for the batch-1 loop, with the
parity decisions recorded in oracle/acceptance.py (greedy = T->0 limit,
textbook residual) and two more:
  * the attention mask is the bottom-right causal rule
    ``col <= (full - S) + row`` (causal_lm.py:400-415); the reference's
    ``_make_causal_mask`` (engine.py:704-710) is all-zero for S != full and is
    not used;
  * ``fill_draft_hole``: after all k drafts are accepted the draft never
    consumed d_{k-1} (speculative.py:76-107), leaving draft KV position
    start+k unwritten; with the flag set (default) the next step first runs
    the draft on d_{k-1}.  ``fill_draft_hole=False`` reproduces the reference.

Weights: every linear / embedding ~ N(0, 0.02) from torch.Generator seeded
with ``seed``, drawn in a fixed order (embed, then per layer q, k, v, o, gate,
up, down), RMSNorm weights 1, q/k/v biases 0; lm_head tied to the embedding
(Qwen2.5-0.5B ties them).

Pinning: the forward reproduces, bit for bit, fp32 logits that the
reference's own CausalLM.forward wrote (tests/golden/make_model_golden.py ->
tests/golden/model_forward_golden.npz: a tiny Qwen2-style config with random
biases and norm weights, a full forward and a cached prefill + verify-style
call; tests/test_oracle_model_golden.py).  Besides, incremental decoding with
the KV cache must equal a full-sequence forward, and greedy speculative
decoding must equal plain greedy decoding of the target for any draft (the
speculative-sampling invariant) -- tests/test_oracle_model.py.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .acceptance import GREEDY_EPS


@dataclass
class ModelConfig:
    """causal_lm.py:77-101 (the fields the verify path uses)."""
    vocab_size: int = 151936
    hidden_size: int = 896
    intermediate_size: int = 4864
    num_hidden_layers: int = 24
    num_attention_heads: int = 14
    num_key_value_heads: int = 2
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    attention_bias: bool = True
    tie_word_embeddings: bool = True

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


QWEN25_05B = ModelConfig()


def init_weights(cfg: ModelConfig, seed: int = 0, dtype=torch.float32):
    """Seeded N(0, 0.02) weights in a fixed draw order (see module doc)."""
    g = torch.Generator().manual_seed(seed)
    H, D = cfg.hidden_size, cfg.head_dim
    Hq, Hkv = cfg.num_attention_heads, cfg.num_key_value_heads

    def n(*shape):
        return (torch.randn(*shape, generator=g) * 0.02).to(dtype)

    w = {"embed": n(cfg.vocab_size, H), "layers": []}
    for _ in range(cfg.num_hidden_layers):
        w["layers"].append({
            "q": n(Hq * D, H), "k": n(Hkv * D, H), "v": n(Hkv * D, H), "o": n(H, Hq * D),
            "gate": n(cfg.intermediate_size, H), "up": n(cfg.intermediate_size, H),
            "down": n(H, cfg.intermediate_size),
            "qb": torch.zeros(Hq * D, dtype=dtype), "kb": torch.zeros(Hkv * D, dtype=dtype),
            "vb": torch.zeros(Hkv * D, dtype=dtype),
            "ln1": torch.ones(H, dtype=dtype), "ln2": torch.ones(H, dtype=dtype),
        })
    w["norm"] = torch.ones(H, dtype=dtype)
    return w


def rms_norm(x, weight, eps):
    """causal_lm.py:142-145."""
    dt = x.dtype
    var = x.float().pow(2).mean(-1, keepdim=True)
    x = x * torch.rsqrt(var + eps)
    return (weight * x).to(dt)


def rope_tables(cfg: ModelConfig, max_pos: int):
    """causal_lm.py:157-164."""
    D = cfg.head_dim
    freqs = 1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2).float() / D))
    t = torch.arange(max_pos).float()
    f = torch.outer(t, freqs)
    return f.cos(), f.sin()


def apply_rope(x, cos, sin, position_ids):
    """causal_lm.py:167-206, batched (B, heads, S, D) layout."""
    dt = x.dtype
    half = x.shape[-1] // 2
    c = torch.cat([cos[position_ids]] * 2, dim=-1).to(dt).unsqueeze(1)
    s = torch.cat([sin[position_ids]] * 2, dim=-1).to(dt).unsqueeze(1)
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return (x * c + rot * s).to(dt)


def causal_mask(seq_len: int, full_len: int, dtype=torch.float32):
    """Bottom-right causal additive mask (causal_lm.py:400-415)."""
    row = torch.arange(seq_len)[:, None]
    col = torch.arange(full_len)[None, :]
    m = torch.where(col <= (full_len - seq_len) + row, 0.0, float("-inf"))
    return m.to(dtype)[None, None]


class CPUCausalLM:
    """Batched forward with a contiguous cache (causal_lm.py:564-583)."""

    def __init__(self, cfg: ModelConfig, weights, num_layers: int | None = None,
                 max_pos: int | None = None):
        self.cfg = cfg
        self.w = weights
        self.num_layers = cfg.num_hidden_layers if num_layers is None else num_layers
        self.cos, self.sin = rope_tables(cfg, max_pos or cfg.max_position_embeddings)

    def new_cache(self, batch: int, max_len: int):
        """NaiveKVCache (kv_cache.py:13-41): per layer (B, Hkv, S_max, D) zeros."""
        c = self.cfg
        return [(torch.zeros(batch, c.num_key_value_heads, max_len, c.head_dim),
                 torch.zeros(batch, c.num_key_value_heads, max_len, c.head_dim))
                for _ in range(self.num_layers)]

    def forward(self, input_ids, position_ids, kv_caches, cache_position, attention_mask):
        c = self.cfg
        B, S = input_ids.shape
        Hq, Hkv, D = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        x = F.embedding(input_ids, self.w["embed"])
        for li in range(self.num_layers):
            L = self.w["layers"][li]
            res = x
            h = rms_norm(x, L["ln1"], c.rms_norm_eps)
            q = F.linear(h, L["q"], L["qb"]).view(B, S, Hq, D).transpose(1, 2)
            k = F.linear(h, L["k"], L["kb"]).view(B, S, Hkv, D).transpose(1, 2)
            v = F.linear(h, L["v"], L["vb"]).view(B, S, Hkv, D).transpose(1, 2)
            q = apply_rope(q, self.cos, self.sin, position_ids)
            k = apply_rope(k, self.cos, self.sin, position_ids)
            kc, vc = kv_caches[li]
            kc[:B, :, cache_position:cache_position + S] = k
            vc[:B, :, cache_position:cache_position + S] = v
            k = kc[:B, :, :cache_position + S]
            v = vc[:B, :, :cache_position + S]
            g = Hq // Hkv
            if g > 1:
                k = k.repeat_interleave(g, dim=1)
                v = v.repeat_interleave(g, dim=1)
            att = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(D)
            if attention_mask is not None:
                att = att + attention_mask
            att = F.softmax(att, dim=-1, dtype=torch.float32).to(q.dtype)
            o = torch.matmul(att, v).transpose(1, 2).contiguous().view(B, S, -1)
            x = F.linear(o, L["o"])
            res = res + x                                   # causal_lm.py:153
            h = rms_norm(res, L["ln2"], c.rms_norm_eps)
            x = res + F.linear(F.silu(F.linear(h, L["gate"])) * F.linear(h, L["up"]), L["down"])
        x = rms_norm(x, self.w["norm"], c.rms_norm_eps)
        return F.linear(x, self.w["embed"])                  # tied lm_head


def greedy_decode(model: CPUCausalLM, prompt: list[int], n_new: int) -> list[int]:
    """Plain (non-speculative) greedy decoding -- the invariant's right side."""
    cache = model.new_cache(1, len(prompt) + n_new + 1)
    ids = torch.tensor([prompt])
    S = len(prompt)
    logits = model.forward(ids, torch.arange(S)[None], cache, 0, causal_mask(S, S))
    out = [int(logits[0, -1].argmax())]
    pos = S
    while len(out) < n_new:
        logits = model.forward(torch.tensor([[out[-1]]]), torch.tensor([[pos]]), cache, pos,
                               causal_mask(1, pos + 1))
        out.append(int(logits[0, -1].argmax()))
        pos += 1
    return out


class CPUSpeculativeDecoder:
    """speculative.py:23-184, batch 1, greedy (T < 1e-6) or stochastic with
    supplied uniforms (a callable ``uniform(n) -> list[float]``)."""

    def __init__(self, draft: CPUCausalLM, target: CPUCausalLM, num_speculative: int,
                 temperature: float = 0.0, fill_draft_hole: bool = True, uniform=None):
        self.draft, self.target = draft, target
        self.k = num_speculative
        self.temperature = temperature
        self.fill_draft_hole = fill_draft_hole
        self.uniform = uniform
        self.stats = {"steps": 0, "proposed": 0, "accepted": 0}

    def generate(self, prompt: list[int], n_new: int) -> list[int]:
        from .acceptance import accept_request
        k = self.k
        greedy = self.temperature < GREEDY_EPS
        S = len(prompt)
        max_len = S + n_new + 2 * k + 2
        tcache = self.target.new_cache(1, max_len)
        dcache = self.draft.new_cache(1, max_len)
        ids = torch.tensor([prompt])
        pos_ids = torch.arange(S)[None]
        mask = causal_mask(S, S)
        logits = self.target.forward(ids, pos_ids, tcache, 0, mask)
        self.draft.forward(ids, pos_ids, dcache, 0, mask)
        first = self._sample(logits[0, -1])
        out = [first]
        pending = [first]       # tokens not yet in the draft cache, oldest first
        start = S               # position of pending[-1]
        while len(out) < n_new:
            # ---- draft: k tokens (first call also consumes a filled hole) ----
            drafts, dlogits = [], []
            cur = pending
            pos0 = start - (len(pending) - 1)
            for i in range(k):
                n_in = len(cur)
                p0 = pos0 if i == 0 else start + i
                ids = torch.tensor([cur])
                lg = self.draft.forward(ids, torch.arange(p0, p0 + n_in)[None], dcache, p0,
                                        causal_mask(n_in, p0 + n_in))[0, -1]
                tok = self._sample(lg)
                drafts.append(tok)
                dlogits.append(lg)
                cur = [tok]
            # ---- verify: [last] + drafts at start .. start+k ----
            vids = torch.tensor([[out[-1]] + drafts])
            tl = self.target.forward(vids, torch.arange(start, start + k + 1)[None], tcache,
                                     start, causal_mask(k + 1, start + k + 1))[0]
            u = self.uniform(k + 1) if not greedy else [0.0] * (k + 1)
            acc, _ = accept_request(tl.numpy(), None if greedy else torch.stack(dlogits).numpy(),
                                    drafts, u, self.temperature)
            n = len(acc)
            self.stats["steps"] += 1
            self.stats["proposed"] += k
            self.stats["accepted"] += n - 1
            out.extend(acc)
            # draft cache holds positions < start + k (d_{k-1} was never consumed)
            if n == k + 1 and self.fill_draft_hole:
                pending = [drafts[-1], acc[-1]]
            else:
                pending = [acc[-1]]
            start += n
        return out[:n_new]

    def _sample(self, logits):
        if self.temperature < GREEDY_EPS:
            return int(logits.argmax())
        from .acceptance import inverse_cdf, softmax64
        p = softmax64(logits.numpy(), self.temperature)
        return inverse_cdf(p, float(self.uniform(1)[0]))[0]
