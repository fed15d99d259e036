"""Speculative decoding -- the reference's host API over the HIP verify step.

Drop-in for nano_sglang/decode/speculative.py:

* ``SpeculativeDecoder(draft_model, target_model, num_speculative=5,
  temperature=1.0, top_p=1.0, top_k=0)`` (:34-48);
* ``speculative_step(input_ids (1,1), start_pos, draft_kv_caches,
  target_kv_caches, make_mask_fn) -> list[int]`` (:50-184): the k draft
  forwards and the one target forward go through the caller's models with
  the reference's batched signature (``forward(input_ids, position_ids,
  kv_caches, cache_position, attention_mask) -> (1, S, V)``); the ratio
  tests, residual resample and bonus run in the fused HIP acceptance kernel
  (``kernels.spec_accept``) instead of the per-position Python loop
  (:130-184);
* ``reset_draft_cache`` (:186-196).

Differences from the literal reference (all documented parity decisions):
greedy (``temperature < 1e-6``) is the T->0 limit of the ratio test; the
resample is the textbook residual ``max(0, p_t - p_d)``; uniforms come from
Philox4x32-10 (``seed``) instead of ``torch.rand``; ``make_mask_fn`` must be
bottom-right causal (use :func:`causal_mask`; the reference engine's
``_make_causal_mask``, engine.py:704-710, is not causal for S != full); and the
draft-cache hole after full acceptance (the draft never consumed d_{k-1}) is
filled on the next call unless ``fill_draft_hole=False``.

``top_k`` / ``top_p`` apply where the reference calls ``sample_token``: the
draft tokens (:95-100) and the bonus token (:174-182), through the HIP sampler
(``kernels.sample``, engine/sampling.py:71-88).  The ratio test uses the
unfiltered ``softmax(logits / T)`` of both models, as the reference does
(:89-92, 104, 134-148); the residual is the textbook one over those
distributions (the reference's filtered fallback, :163-169, is only reached
when the residual is empty, which the textbook residual never is after a
rejection).

``generate_batch`` is additive API: batched speculative decoding on the paged
KV cache (``engine.spec_engine.SpecEngine``) for a target built by
``model.causal_lm.CausalLM``.
"""

from __future__ import annotations

import torch

from .. import kernels


def causal_mask(seq_len: int, full_len: int, dtype=torch.float32, device="cuda") -> torch.Tensor:
    """Bottom-right causal additive mask (nano_sglang/model/causal_lm.py:400-415)."""
    row = torch.arange(seq_len, device=device)[:, None]
    col = torch.arange(full_len, device=device)[None, :]
    return torch.where(col <= (full_len - seq_len) + row, 0.0, float("-inf")).to(dtype)[None, None]


class SpeculativeDecoder:
    def __init__(self, draft_model, target_model, num_speculative: int = 5,
                 temperature: float = 1.0, top_p: float = 1.0, top_k: int = 0, seed: int = 0,
                 fill_draft_hole: bool = True):
        if not 0.0 < top_p or top_p != top_p:
            raise ValueError(f"top_p {top_p} must be in (0, 1] (1 = off)")
        self.draft_model = draft_model
        self.target_model = target_model
        self.num_speculative = num_speculative
        self.temperature = temperature
        self.top_p = top_p
        self.top_k = top_k
        self.seed = seed
        self.fill_draft_hole = fill_draft_hole
        self._offset = [0, 0]      # Philox offsets: stream 0 acceptance, 1 draft sampling
        self._unconsumed = None    # (token, position) the draft cache still lacks

    def _uniforms(self, stream: int, n: int, device) -> torch.Tensor:
        u = kernels.philox_uniform(self.seed, stream, self._offset[stream], n, device)
        self._offset[stream] += n
        return u

    @staticmethod
    def _logits_dtype(x: torch.Tensor) -> torch.Tensor:
        return x if x.dtype in (torch.bfloat16, torch.float32) else x.float()

    def _filtered(self) -> bool:
        return self.temperature >= 1e-6 and (self.top_k > 0 or self.top_p < 1.0)

    def _sample(self, row: torch.Tensor) -> torch.Tensor:
        """One token from a (1, V) logits row (sample_token, sampling.py:25-50):
        argmax, or an inverse-CDF draw from softmax(row / T) after top-k / top-p."""
        row = self._logits_dtype(row)
        greedy = self.temperature < 1e-6
        u = None if greedy else self._uniforms(1, 1, row.device).view(1, 1)
        if self._filtered():
            return kernels.sample(row.reshape(1, -1), self.temperature, self.top_k, self.top_p,
                                  u.view(1))
        _, em, _ = kernels.spec_accept(row.view(1, 1, -1).contiguous(), None, None, u,
                                       self.temperature)
        return em[:, 0]

    @torch.inference_mode()
    def speculative_step(self, input_ids: torch.Tensor, start_pos: int, draft_kv_caches,
                         target_kv_caches, make_mask_fn) -> list[int]:
        """One propose-verify step; returns the 1..k+1 emitted token ids."""
        k = self.num_speculative
        dev = input_ids.device
        greedy = self.temperature < 1e-6
        # ---- draft: k tokens (speculative.py:76-107) ----
        cur = input_ids
        pos = start_pos
        if self.fill_draft_hole and self._unconsumed is not None \
                and self._unconsumed[1] == start_pos - 1:
            cur = torch.cat([torch.tensor([[self._unconsumed[0]]], device=dev), input_ids], 1)
            pos = start_pos - 1
        self._unconsumed = None
        drafts, dlogits = [], []
        for i in range(k):
            n_in = cur.shape[1]
            logits = self.draft_model(
                input_ids=cur, position_ids=torch.arange(pos, pos + n_in, device=dev)[None],
                kv_caches=draft_kv_caches, cache_position=pos,
                attention_mask=make_mask_fn(n_in, pos + n_in))
            row = logits[:, -1, :]
            tok = self._sample(row)
            drafts.append(tok)
            dlogits.append(self._logits_dtype(row))
            pos += n_in
            cur = tok.view(1, 1)
        # ---- verify: one target forward over k+1 tokens (speculative.py:109-128) ----
        verify_ids = torch.cat([input_ids.view(1, 1)] + [d.view(1, 1) for d in drafts], 1)
        tl = self.target_model(
            input_ids=verify_ids,
            position_ids=torch.arange(start_pos, start_pos + k + 1, device=dev)[None],
            kv_caches=target_kv_caches, cache_position=start_pos,
            attention_mask=make_mask_fn(k + 1, start_pos + k + 1))
        tl = self._logits_dtype(tl).contiguous()
        dl = None if greedy else torch.stack(dlogits, 1).to(tl.dtype).contiguous()
        u = None if greedy else self._uniforms(0, k + 1, dev).view(1, k + 1)
        bonus = None
        if self._filtered():    # speculative.py:174-182: sample_token with the filters
            bonus = kernels.sample(tl[:, k], self.temperature, self.top_k, self.top_p, u[:, k])
        n, emitted, _ = kernels.spec_accept(tl, dl, torch.stack(drafts, 1), u, self.temperature,
                                            bonus_tokens=bonus)
        n = int(n.item())
        out = emitted[0, :n].tolist()
        if n == k + 1:
            self._unconsumed = (int(drafts[-1].item()), start_pos + k)
        return out

    def reset_draft_cache(self, draft_kv_caches, accepted_len: int, start_pos: int) -> None:
        """Contiguous caches need no rollback: positions past the accepted
        prefix are overwritten by the next step (speculative.py:186-196).  The
        paged path rolls back through PagedKVCache.truncate."""
        return None

    def generate_batch(self, prompts: list[list[int]], max_new_tokens: list[int],
                       num_blocks: int = 8000, block_size: int = 16, draft_layers: int = 4):
        """Batched speculative decoding on the paged KV cache (additive API)."""
        from ..engine.spec_engine import SpecEngine
        eng = SpecEngine(self.target_model, draft_layers=draft_layers,
                         num_speculative=self.num_speculative, num_blocks=num_blocks,
                         block_size=block_size, temperature=self.temperature, seed=self.seed,
                         top_k=self.top_k, top_p=self.top_p)
        out = eng.generate(prompts, max_new_tokens)
        self.last_stats = eng.stats
        return out
