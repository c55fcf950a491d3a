"""Oracle: Huginn forward and per-request CDB decoding in numpy (test infrastructure).

Restates, one request at a time:
  * the Huginn block (huginn/modeling_huginn.py:223-338): sandwich norms
    x1 = norm_2(attn(norm_1(x)) + x), out = norm_4(mlp(norm_3(x1)) + x1); fused
    Wqkv; the per-head qk_bias added (rounded) before interleaved-pair RoPE in
    fp32 (theta = rope_base, one rounding); causal attention over the request's
    KV; SwiGLU MLP from one fused gate/up projection;
  * the stages (:399-463): prelude on sqrt(n_embd)-scaled embeddings, the core
    step adapter(cat(state, injection)) -> core blocks, coda ln_f -> blocks -> ln_f,
    tied LM head; zero initial state;
  * full-depth prefill writing prelude, core-slot and coda KV, first token from
    the last prompt position (cdb/continuous_api.py:995-1088);
  * CDB decode of each later token (cdb/adapters/huginn.py:109-189): prelude with
    attention at the token's position, recurrent steps until the exit decision
    (replayed 0-based depth; or the latent difference ||s_r - s_{r-1}|| /
    max(||s_r||, 1e-9) against a direct threshold, huginn/exit_gates.py:33-40,
    cdb/exit_policy.py:150-169, consumed one step late on the delayed horizon),
    the coda with attention at the token's position, greedy argmax.

Pinned by tests/test_oracle_huginn.py: an independent float64 torch forward
built on torch's scaled_dot_product_attention (library routine) and complex
multiplication for the rotary pairs, and the staged-vs-monolithic property
(full-depth prefill of prompt[:-1] plus a full-depth decode of the last token
gives the monolithic forward's logits).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .bf16 import rounder
from .paged_attention import apply_rope
from .stage import rmsnorm, silu_mul


@dataclass
class HuginnOracleOutput:
    tokens: list[int]
    exit_depths: list[int] = field(default_factory=list)
    signals: list[list[float]] = field(default_factory=list)


def huginn_rope_tables(head_dim: int, theta: float, max_positions: int) -> tuple[np.ndarray, np.ndarray]:
    """fp32 cos/sin of position * inv_freq (huginn/modeling_huginn.py:150-175)."""

    inv = (1.0 / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim))))
    inv = inv.astype(np.float32)
    freqs = (np.arange(max_positions, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


class HuginnOracle:
    def __init__(self, weights: dict[str, np.ndarray], *, n_embd: int, n_heads: int, n_prelude: int, n_core: int,
                 n_coda: int, rope_base: float, eps: float, dtype: str = "f32", max_positions: int = 4096,
                 accumulate: str = "f32") -> None:
        """``accumulate`` is the dot-product precision of the projections ("f32", like the GPU
        GEMMs, or "f64"); their results are rounded to ``dtype`` either way, so the two settings
        are two valid implementations whose spread is the size of accumulation-order noise."""

        self.w = {k: np.asarray(v, dtype=np.float32) for k, v in weights.items()}
        self.acc = np.float64 if accumulate == "f64" else np.float32
        self._w64: dict[int, np.ndarray] = {}
        self.E, self.H = n_embd, n_heads
        self.D = n_embd // n_heads
        self.n_prelude, self.n_core, self.n_coda = n_prelude, n_core, n_coda
        self.eps = eps
        self.dtype = dtype
        self.rnd = rounder(dtype)
        self.cos, self.sin = huginn_rope_tables(self.D, rope_base, max_positions)
        self.embed_scale = float(np.sqrt(n_embd))

    # -- pieces ------------------------------------------------------------------------------------------------
    def _mm(self, x: np.ndarray, weight: np.ndarray) -> np.ndarray:
        if self.acc is np.float32:
            return self.rnd(np.asarray(x, np.float32) @ weight.T)
        wide = self._w64.get(id(weight))
        if wide is None:
            wide = self._w64[id(weight)] = weight.astype(np.float64)
        return self.rnd((np.asarray(x, np.float64) @ wide.T).astype(np.float32))

    def _norm(self, x: np.ndarray, name: str) -> np.ndarray:
        return rmsnorm(x, self.w[name], self.eps, self.dtype)

    def _attend(self, kv: np.ndarray, layer: int, q: np.ndarray, k: np.ndarray, v: np.ndarray,
                positions: np.ndarray, q_bias: np.ndarray | None, k_bias: np.ndarray | None) -> np.ndarray:
        cos, sin = self.cos[positions], self.sin[positions]
        if q_bias is not None:
            q = self.rnd(q + q_bias[None])
            k = self.rnd(k + k_bias[None])
        qr = apply_rope(q, cos, sin, 2, self.dtype)
        kr = apply_rope(k, cos, sin, 2, self.dtype)
        kv[layer, 0, positions] = kr
        kv[layer, 1, positions] = v
        end = int(positions[-1]) + 1
        keys = kv[layer, 0, :end].astype(np.float64)
        vals = kv[layer, 1, :end].astype(np.float64)
        out = np.zeros(qr.shape, dtype=np.float32)
        mask = np.arange(end)[None, :] <= positions[:, None]
        for h in range(self.H):
            s = qr[:, h].astype(np.float64) @ keys[:, h].T * self.D ** -0.5
            s = np.where(mask, s, -np.inf)
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[:, h] = (p @ vals[:, h]).astype(np.float32)
        return self.rnd(out)

    def _block(self, prefix: str, x: np.ndarray, kv: np.ndarray, layer: int, positions: np.ndarray) -> np.ndarray:
        n = x.shape[0]
        qkv = self._mm(self._norm(x, prefix + "norm_1.weight"), self.w[prefix + "attn.Wqkv.weight"])
        q = qkv[:, :self.E].reshape(n, self.H, self.D)
        k = qkv[:, self.E:2 * self.E].reshape(n, self.H, self.D)
        v = qkv[:, 2 * self.E:].reshape(n, self.H, self.D)
        bias = self.w.get(prefix + "attn.qk_bias")
        qb, kb = (bias[0, 0], bias[1, 0]) if bias is not None else (None, None)
        a = self._attend(kv, layer, q, k, v, positions, qb, kb)
        o = self._mm(a.reshape(n, self.E), self.w[prefix + "attn.proj.weight"])
        x1 = self._norm(self.rnd(o + x), prefix + "norm_2.weight")
        m = self._mm(silu_mul(self._mm(self._norm(x1, prefix + "norm_3.weight"), self.w[prefix + "mlp.fc.weight"]),
                              self.dtype), self.w[prefix + "mlp.proj.weight"])
        return self._norm(self.rnd(m + x1), prefix + "norm_4.weight")

    def prelude(self, tokens: list[int], kv: np.ndarray, positions: np.ndarray) -> np.ndarray:
        x = self.rnd(self.rnd(self.w["transformer.wte.weight"][np.asarray(tokens)]) * np.float32(self.embed_scale))
        for i in range(self.n_prelude):
            x = self._block(f"transformer.prelude.{i}.", x, kv, i, positions)
        return x

    def core_step(self, state: np.ndarray, injection: np.ndarray, kv: np.ndarray, slot: int,
                  positions: np.ndarray) -> np.ndarray:
        x = self._mm(np.concatenate([state, injection], axis=-1), self.w["transformer.adapter.weight"])
        base = self.n_prelude + slot * self.n_core
        for i in range(self.n_core):
            x = self._block(f"transformer.core_block.{i}.", x, kv, base + i, positions)
        return x

    def coda(self, state: np.ndarray, kv: np.ndarray, num_slots: int, positions: np.ndarray) -> np.ndarray:
        x = self._norm(state, "transformer.ln_f.weight")
        base = self.n_prelude + num_slots * self.n_core
        for i in range(self.n_coda):
            x = self._block(f"transformer.coda.{i}.", x, kv, base + i, positions)
        return self._norm(x, "transformer.ln_f.weight")

    def logits(self, hidden: np.ndarray) -> np.ndarray:
        return self._mm(hidden[None, :], self.w["lm_head.weight"])[0]

    def latent_diff(self, state: np.ndarray, prev: np.ndarray) -> float:
        """R(R(||R(s - p)||) / max(R(||s||), R(1e-9))) (huginn/exit_gates.py:33-40 on model-dtype tensors)."""

        d = self.rnd(state.astype(np.float32) - prev.astype(np.float32)).astype(np.float64)
        num = self.rnd(np.array([np.sqrt((d * d).sum())], np.float32))[0]
        floor = float(self.rnd(np.array([1e-9], np.float32))[0])
        den = max(float(self.rnd(np.array([np.sqrt((state.astype(np.float64) ** 2).sum())], np.float32))[0]), floor)
        return float(self.rnd(np.array([num / den], np.float32))[0])

    # -- request-level ---------------------------------------------------------------------------------------------
    def num_cache_layers(self, num_slots: int) -> int:
        return self.n_prelude + num_slots * self.n_core + self.n_coda

    def prefill_hidden(self, prompt: list[int], kv: np.ndarray, *, steps: int, slot_of, num_slots: int) -> np.ndarray:
        pos = np.arange(len(prompt))
        injection = self.prelude(prompt, kv, pos)
        state = np.zeros_like(injection)
        for step in range(steps):
            state = self.core_step(state, injection, kv, slot_of(step), pos)
        return self.coda(state, kv, num_slots, pos)

    def generate(self, prompt: list[int], max_new_tokens: int, *, max_steps: int, kv_policy: str = "single",
                 exit_depths: list[int] | None = None, threshold: float | None = None, min_steps: int = 1,
                 delayed: bool = False, eos_token_id: int | None = None, forced_tokens: list[int] | None = None,
                 hidden_trace: list | None = None) -> HuginnOracleOutput:
        """Greedy CDB decode of one request. ``forced_tokens`` feeds the given tokens back instead
        of the oracle's own (teacher forcing; ``tokens`` still records the oracle's argmax), and
        ``hidden_trace`` collects (decode token index j >= 1, loop step, recurrent state after the
        step)."""

        num_slots = {"single": 1, "depth_indexed": max_steps, "last_exited": max_steps}[kv_policy]

        def slot_of(step: int) -> int:
            return 0 if kv_policy == "single" else step

        total = len(prompt) + max_new_tokens + 1
        kv = np.zeros((self.num_cache_layers(num_slots), 2, total, self.H, self.D), dtype=np.float32)
        h = self.prefill_hidden(prompt, kv, steps=max_steps, slot_of=slot_of, num_slots=num_slots)
        token = int(np.argmax(self.logits(h[-1])))
        out = HuginnOracleOutput(tokens=[token])
        if forced_tokens is not None:
            token = forced_tokens[0]
        pos = len(prompt)
        while len(out.tokens) < max_new_tokens and token != eos_token_id:
            k_idx = len(out.tokens) - 1
            depth = None if exit_depths is None else exit_depths[k_idx]
            p = np.array([pos])
            injection = self.prelude([token], kv, p)
            state = np.zeros_like(injection)
            exit_step = max_steps - 1
            pending: float | None = None
            signals: list[float] = []
            for step in range(max_steps):
                prev = state
                state = self.core_step(state, injection, kv, slot_of(step), p)
                if hidden_trace is not None:
                    hidden_trace.append((k_idx + 1, step, state[0].copy()))
                if step == max_steps - 1:
                    break
                if depth is not None:
                    if (not delayed and step >= depth) or (delayed and step >= 1 and step - 1 >= depth):
                        exit_step = step
                        break
                    continue
                if threshold is None:
                    continue
                signal = self.latent_diff(state[0], prev[0])
                signals.append(signal)
                consumed, source = (signal, step) if not delayed else (pending, step - 1)
                pending = signal
                if consumed is None:
                    continue
                if source + 1 >= min_steps and consumed < threshold:
                    exit_step = step
                    break
            out.exit_depths.append(exit_step)
            out.signals.append(signals)
            if kv_policy == "last_exited" and exit_step < max_steps - 1:
                for s in range(exit_step + 1, max_steps):
                    for i in range(self.n_core):
                        src = self.n_prelude + exit_step * self.n_core + i
                        kv[self.n_prelude + s * self.n_core + i, :, pos] = kv[src, :, pos]
            h = self.coda(state, kv, num_slots, p)
            token = int(np.argmax(self.logits(h[0])))
            out.tokens.append(token)
            if forced_tokens is not None:
                token = forced_tokens[len(out.tokens) - 1]
            pos += 1
        return out
