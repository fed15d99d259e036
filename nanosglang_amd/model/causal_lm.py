"""Qwen2 / Llama decoder on one MI355X for the speculative verify path.

Mirrors nano_sglang/model/causal_lm.py where the verify path needs it:
``ModelConfig`` (:77-101), pre-norm decoder layers with fused residual +
RMSNorm (:474-532), SwiGLU MLP (:481-482), tied embedding / lm_head, and the
packed forward ``forward_packed(input_ids, positions, kv_cache, attn_wrapper,
write_indices, logit_indices)`` of the FlashInfer path (:585-646), where each
layer writes its K/V into the paged pool and runs paged attention
(:329-342).

MI355X-side choices:
* q/k/v are one fused GEMM (and gate/up another, with the SwiGLU gate in its
  epilogue); at decode / verify row counts (<= 160) every linear layer runs
  the HIP weight-streaming kernel ``kernels.linear``, at prefill sizes
  hipBLASLt;
* RoPE + KV-slot write (with the reference's bf16 rounding order) is the
  epilogue of the q/k/v projection at decode / verify row counts
  (``kernels.linear_rope_kv``: the projection never reaches HBM) and its own
  HIP kernel (``kernels.rope_kv_write``) after a prefill GEMM; attention is
  the HIP verify-attention kernel behind
  ``BatchPrefillWithPagedKVCacheWrapper``;
* RMSNorm (and residual add + RMSNorm) and the SwiGLU gate are HIP kernels
  with the reference's fp32-variance arithmetic (:142-154, :482); with bf16
  weights, hidden <= 1024 and at most 160 rows (decode / verify steps), the
  two norms of every layer run inside the linears around them instead: the
  norm weight is folded into the q/k/v and gate/up weight columns once, the
  o_proj and down_proj kernels add their result to the residual stream and
  write the rows' partial sums of squares, and the q/k/v and gate/up kernels
  scale each row by rsqrt(mean(x^2) + eps) before their epilogues -- two
  launches fewer per layer; the final norm folds into the lm_head the same
  way (``kernels.lm_head_fold``) when every row's logits or tokens are
  wanted;
* a draft made of the first ``n`` layers plus the shared embedding, final
  norm and lm_head is ``forward_packed(..., num_layers=n)`` on the same
  weights.

Random init (no checkpoints offline): every linear and embedding weight
~ N(0, 0.02), RMSNorm weights 1, q/k/v biases 0, drawn on the device from a
seeded generator; or pass ``weights`` (the layout of a dict of fp32 tensors
with keys embed / layers[q,k,v,o,gate,up,down,qb,kb,vb,ln1,ln2] / norm).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .. import kernels


@dataclass
class ModelConfig:
    """nano_sglang/model/causal_lm.py:77-101 (defaults: Qwen2.5-0.5B shape)."""
    model_type: str = "qwen2"
    vocab_size: int = 151936
    hidden_size: int = 896
    intermediate_size: int = 4864
    num_hidden_layers: int = 24
    num_attention_heads: int = 14
    num_key_value_heads: int = 2
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = True
    attention_bias: bool = True

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


def rope_tables(cfg: ModelConfig, device):
    """causal_lm.py:157-164, computed in fp32 on the host then moved."""
    D = cfg.head_dim
    freqs = 1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2).float() / D))
    t = torch.arange(cfg.max_position_embeddings).float()
    f = torch.outer(t, freqs)
    return f.cos().contiguous().to(device), f.sin().contiguous().to(device)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """causal_lm.py:142-145: fp32 variance, x * rsqrt, weight * x, cast back."""
    dt = x.dtype
    var = x.float().pow(2).mean(-1, keepdim=True)
    return (weight * (x * torch.rsqrt(var + eps))).to(dt)


class CausalLM:
    def __init__(self, config: ModelConfig, device="cuda", dtype=torch.bfloat16, seed: int = 0,
                 weights: dict | None = None):
        self.config = c = config
        self.device = torch.device(device)
        self.dtype = dtype
        H, D = c.hidden_size, c.head_dim
        Hq, Hkv, I = c.num_attention_heads, c.num_key_value_heads, c.intermediate_size
        if weights is None:
            g = torch.Generator(device=self.device).manual_seed(seed)

            def n(*shape):
                return (torch.randn(*shape, generator=g, device=self.device,
                                    dtype=torch.float32) * 0.02).to(dtype)

            def z(*shape):
                return torch.zeros(*shape, device=self.device, dtype=dtype)

            def o(*shape):
                return torch.ones(*shape, device=self.device, dtype=dtype)

            self.embed = n(c.vocab_size, H)
            self.layers = []
            for _ in range(c.num_hidden_layers):
                self.layers.append({
                    "qkv": torch.cat([n(Hq * D, H), n(Hkv * D, H), n(Hkv * D, H)]),
                    "qkv_b": z((Hq + 2 * Hkv) * D), "o": n(H, Hq * D),
                    "gate_up": torch.cat([n(I, H), n(I, H)]), "down": n(H, I),
                    "ln1": o(H), "ln2": o(H)})
            self.norm = o(H)
        else:
            def d(t):
                return t.to(self.device, dtype)

            self.embed = d(weights["embed"])
            self.layers = []
            for L in weights["layers"]:
                self.layers.append({
                    "qkv": d(torch.cat([L["q"], L["k"], L["v"]])),
                    "qkv_b": d(torch.cat([L["qb"], L["kb"], L["vb"]])), "o": d(L["o"]),
                    "gate_up": d(torch.cat([L["gate"], L["up"]])), "down": d(L["down"]),
                    "ln1": d(L["ln1"]), "ln2": d(L["ln2"])})
            self.norm = d(weights["norm"])
        self.lm_head = self.embed  # tie_word_embeddings
        self.lm_head_g = None
        self.rope_cos, self.rope_sin = rope_tables(c, self.device)
        self._fold = self._fold_norm_weights()
        self.last_forward_folded = False

    def _fold_norm_weights(self) -> bool:
        """RMSNorm folded into the linears after it (bf16 weights, hidden a
        multiple of 16 and at most 1024): each layer gets copies of its q/k/v
        and gate/up weights with its norm weight folded into their columns,
        ``qkv_g`` / ``gate_up_g`` = bf16(w_ln[k] * W[n, k]), and the lm_head
        the final norm's weight (``lm_head_g``); the forward then runs the
        folded path (``forward_packed``).  Returns whether it did."""
        H = self.config.hidden_size
        if self.dtype != torch.bfloat16 or H % 16 or H > 1024:
            return False
        for L in self.layers:
            L["qkv_g"] = (L["qkv"].float() * L["ln1"].float()[None, :]).to(torch.bfloat16)
            L["gate_up_g"] = (L["gate_up"].float() * L["ln2"].float()[None, :]).to(torch.bfloat16)
        # the final norm folded into the lm_head the same way (the tied
        # embedding itself when the norm weight is all ones)
        if bool((self.norm == 1).all()):
            self.lm_head_g = self.lm_head
        else:
            self.lm_head_g = torch.empty_like(self.lm_head)
            for r0 in range(0, self.lm_head.shape[0], 16384):
                rows = self.lm_head[r0:r0 + 16384].float() * self.norm.float()[None, :]
                self.lm_head_g[r0:r0 + 16384] = rows.to(torch.bfloat16)
        self._ones = torch.ones(H, device=self.device, dtype=torch.bfloat16)
        return True

    def quantize_fp8(self, resident_dequant: bool = False) -> "CausalLM":
        """FP8 (E4M3) weights for every decoder layer's q/k/v, o_proj,
        gate/up and down_proj, one per-tensor scale each (FP8Linear.from_linear,
        nano_sglang/decode/quantization.py:54-75); embeddings, lm_head and
        norms stay bf16, as the reference's default skip list keeps them
        (:220-221).  In place; returns self.

        ``resident_dequant``: also keep the dequantised bf16 weights
        (``dequant_fp8``, bit-identical to dequantising per call) for the
        row counts that go to the library GEMM, so those calls read 2 bytes
        per weight instead of dequantising first (3 more); the FP8 bytes
        still serve the weight-streaming kernel.  Costs 2 bytes per weight of
        HBM."""
        from .quantization import fp8_quantize_rows
        c = self.config
        # FP8 weights keep the norms as kernels of their own (a per-row FP8
        # scale cannot absorb a per-column norm weight)
        self._fold = False
        self.lm_head_g = None
        for L in self.layers:
            L.pop("qkv_g", None)
            L.pop("gate_up_g", None)
        Hq, Hkv, D, I = (c.num_attention_heads, c.num_key_value_heads, c.head_dim,
                         c.intermediate_size)
        for L in self.layers:
            if "qkv_s" in L:
                continue
            L["qkv"], L["qkv_s"] = fp8_quantize_rows(L["qkv"], [Hq * D, Hkv * D, Hkv * D])
            L["o"], L["o_s"] = fp8_quantize_rows(L["o"], [L["o"].shape[0]])
            L["gate_up"], L["gate_up_s"] = fp8_quantize_rows(L["gate_up"], [I, I])
            L["down"], L["down_s"] = fp8_quantize_rows(L["down"], [L["down"].shape[0]])
        if resident_dequant:
            for L in self.layers:
                for n in ("qkv", "o", "gate_up", "down"):
                    L[n + "_d"] = kernels.dequant_fp8(L[n], L[n + "_s"])
        return self

    def keys_supported(self, T: int) -> bool:
        """Whether a forward over T rows can hand its greedy tokens to the
        next one as argmax keys (``forward_packed(argmax_keys_out=...)``,
        ``ids_keys``): the folded norms, the bf16 embedding lookup and the
        folded lm_head all take T rows."""
        c = self.config
        return (self._fold and T <= kernels._lib().nsg_linear_max_rows()
                and self.embed.dtype == torch.bfloat16 and c.hidden_size % 16 == 0
                and kernels.lm_head_fold_supported(T, c.vocab_size, c.hidden_size,
                                                   c.hidden_size // 16))

    @property
    def num_layers(self) -> int:
        return self.config.num_hidden_layers

    @torch.inference_mode()
    def forward_packed(self, input_ids: torch.Tensor, positions: torch.Tensor, kv_cache,
                       attn_wrapper, write_indices: torch.Tensor,
                       logit_indices: torch.Tensor | None = None,
                       num_layers: int | None = None, argmax_out: torch.Tensor | None = None,
                       argmax_ws=None, argmax_logits: torch.Tensor | None = None,
                       argmax_keys_out: torch.Tensor | None = None,
                       ids_keys: tuple | None = None):
        """Packed forward over ``T`` tokens of several requests.

        kv_cache: (k_cache, v_cache) pools (L, N, P, Hkv, D); attn_wrapper: a
        planned ``BatchPrefillWithPagedKVCacheWrapper``; write_indices: int64
        flat slots (T,).  Returns logits (len(logit_indices) or T, V), or,
        with ``argmax_out`` (int64, one per row), each row's greedy token
        written there (``kernels.linear_argmax``: the logits are never
        stored); ``argmax_logits`` (T, V) bf16 then also receives the logits
        those tokens are the argmax of (same kernel and rounding; for tests
        and traces).  With ``argmax_keys_out`` (a device buffer) instead, only
        the rows' argmax keys are written there and the keys per row returned
        (``kernels.lm_head_fold``), for the next call's ``ids_keys`` =
        (keys, key_cols, j): column j of ``input_ids`` (B, J) then receives
        those greedy tokens inside the embedding lookup -- no reduction
        launch between the two forwards.  Both need ``keys_supported``."""
        c = self.config
        Hq, Hkv, D, I = (c.num_attention_heads, c.num_key_value_heads, c.head_dim,
                         c.intermediate_size)
        k_pool, v_pool = kv_cache
        nl = self.num_layers if num_layers is None else num_layers
        eps = c.rms_norm_eps
        T = input_ids.numel()
        folded = self._fold and T <= kernels._lib().nsg_linear_max_rows()
        self.last_forward_folded = folded     # which norm path the call took
        ssa = None
        if (argmax_keys_out is not None or ids_keys is not None) and (
                not self.keys_supported(T)
                or (argmax_keys_out is not None and logit_indices is not None)):
            raise ValueError(f"argmax keys need the folded forward with the folded lm_head "
                             f"at {T} rows")
        if self.embed.dtype == torch.bfloat16 and c.hidden_size % 16 == 0:
            # causal_lm.py:613 -- ids may be any (T,) or (B, J) view; with the
            # folded norms the lookup also writes the first partial sums
            if folded:
                ssa = torch.empty(c.hidden_size // 16, T, dtype=torch.float32,
                                  device=self.device)
            residual = kernels.embed_rows(input_ids, self.embed, sumsq_out=ssa, keys=ids_keys)
        else:
            residual = F.embedding(input_ids.reshape(-1), self.embed)
        # residual: owned, updated in place below
        if folded:
            # folded norms: residual += o_proj(.) and += down_proj(.) in those
            # kernels, which also write the rows' partial sums of squares
            # (ssb, ssa); q/k/v and gate/up read them (causal_lm.py:505-531)
            if ssa is None:
                ssa = kernels.row_sumsq(residual)
            ssb = torch.empty_like(ssa)
            for li in range(nl):
                L = self.layers[li]
                q = kernels.linear_rope_kv(residual, L["qkv_g"], L["qkv_b"], Hq, Hkv, D,
                                           positions, self.rope_cos, self.rope_sin,
                                           write_indices, k_pool[li], v_pool[li],
                                           sumsq_in=ssa, norm_eps=eps)
                attn = attn_wrapper.run(q, (k_pool[li], v_pool[li]))
                kernels.linear(attn.view(-1, Hq * D), L["o"], residual=residual, sumsq_out=ssb)
                g = kernels.linear(residual, L["gate_up_g"], swiglu=True, sumsq_in=ssb,
                                   norm_eps=eps)
                kernels.linear(g, L["down"], residual=residual, sumsq_out=ssa)
            if logit_indices is None and kernels.lm_head_fold_supported(
                    T, c.vocab_size, c.hidden_size, ssa.shape[0]):
                # the final norm folded into the lm_head (causal_lm.py:643-645):
                # the residual rows and their partial sums go straight in
                if argmax_keys_out is not None:
                    if argmax_logits is not None:
                        kernels.lm_head_fold(residual, self.lm_head_g, ssa, eps,
                                             out=argmax_logits)
                    return kernels.lm_head_fold(residual, self.lm_head_g, ssa, eps,
                                                keys_out=argmax_keys_out)
                if argmax_out is not None:
                    if argmax_logits is not None:
                        kernels.lm_head_fold(residual, self.lm_head_g, ssa, eps,
                                             out=argmax_logits)
                    return kernels.lm_head_fold(residual, self.lm_head_g, ssa, eps,
                                                argmax_out=argmax_out, workspace=argmax_ws)
                return kernels.lm_head_fold(residual, self.lm_head_g, ssa, eps)
            h = kernels.rmsnorm(residual, self.norm, eps)
        else:
            # separate norm kernels; with folded weights (many rows: prefill)
            # the norms run with unit weights
            qkv_k, gu_k = ("qkv_g", "gate_up_g") if self._fold else ("qkv", "gate_up")
            x = None
            for li in range(nl):
                L = self.layers[li]
                ln1, ln2 = (self._ones, self._ones) if self._fold else (L["ln1"], L["ln2"])
                # residual += x (causal_lm.py:505, 531), then RMSNorm -- one kernel
                h = kernels.rmsnorm(residual if x is None else x, ln1, eps,
                                    residual=None if x is None else residual)
                q = kernels.linear_rope_kv(h, L[qkv_k], L["qkv_b"], Hq, Hkv, D, positions,
                                           self.rope_cos, self.rope_sin, write_indices,
                                           k_pool[li], v_pool[li], w_scale=L.get("qkv_s"),
                                           w_dequant=L.get("qkv_d"))
                attn = attn_wrapper.run(q, (k_pool[li], v_pool[li]))
                x = kernels.linear(attn.view(-1, Hq * D), L["o"], w_scale=L.get("o_s"),
                                   w_dequant=L.get("o_d"))
                h = kernels.rmsnorm(x, ln2, eps, residual=residual)   # causal_lm.py:147-154
                x = kernels.linear(kernels.linear(h, L[gu_k], swiglu=True,
                                                  w_scale=L.get("gate_up_s"),
                                                  w_dequant=L.get("gate_up_d")),
                                   L["down"], w_scale=L.get("down_s"),
                                   w_dequant=L.get("down_d"))
            h = kernels.rmsnorm(x, self.norm, eps, residual=residual)
        if logit_indices is not None:
            h = h[logit_indices]
        if argmax_out is not None:
            if argmax_logits is not None:
                kernels.linear(h, self.lm_head, out=argmax_logits, force=True)
            return kernels.linear_argmax(h, self.lm_head, out=argmax_out, workspace=argmax_ws)
        return kernels.linear(h, self.lm_head)
