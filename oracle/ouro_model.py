"""Oracle: Ouro forward and per-request CDB decoding in numpy (test infrastructure).

Restates, one request at a time:
  * the Ouro layer stack (ouro/modeling_ouro.py:377-503): RMSNorm sandwiches,
    split-half RoPE with model-dtype cos/sin, causal attention over the
    request's KV, SwiGLU MLP, the final norm after each loop step
    (:601-627, cdb/adapters/ouro.py:214-264);
  * full-depth prefill: every loop step ut writes its KV into cache slot
    slot(ut) (ouro/modeling_ouro.py:630-724, kv_cache_policy.py:84-128) and the
    last prompt position samples the first token greedily;
  * CDB decode of each later token: prelude = embedding, recurrent steps until
    the exit decision (replayed 0-based depth, or the hazard-CDF gate with the
    forced exit at the last step; continuous_api.py:1671-1724), the exit-KV
    copy into deeper slots under ``last_exited`` (:1225-1245), coda = LM head +
    argmax (cdb/model_runner.py:1036-1062).
Because every request's math depends only on its own KV and exit depths, the
batched engine must produce the same token streams whatever its batching.

Pinned by tests/test_oracle_model.py: a torch re-implementation of the layer
with torch's scaled_dot_product_attention (library routine), and the
reference's own consistency property (staged prefill + decode of the last token
equals the monolithic full-depth forward; tests/continuous_depth_batching/
test_ouro_cdb_staged_api.py:24-52).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .bf16 import rounder
from .paged_attention import apply_rope, rope_tables
from .stage import gate_logits, ouro_sandwich, rmsnorm, sigmoid_f32, silu_mul


@dataclass
class OracleOutput:
    tokens: list[int]
    exit_depths: list[int] = field(default_factory=list)
    exit_copies: int = 0


class OuroOracle:
    def __init__(self, weights: dict[str, np.ndarray], *, num_layers: int, num_heads: int, num_kv_heads: int,
                 head_dim: int, rope_theta: float, eps: float, dtype: str = "f32", max_positions: int = 4096,
                 gate: str = "early_exit", accumulate: str = "f32") -> None:
        """``accumulate`` is the dot-product precision of the projections ("f32", like the GPU
        GEMMs, or "f64"); their results are rounded to ``dtype`` either way. Two settings give two
        valid implementations, whose spread is the size of bf16 accumulation-order noise."""

        self.w = {k: np.asarray(v, dtype=np.float32) for k, v in weights.items()}
        self.L, self.H, self.Hkv, self.D = num_layers, num_heads, num_kv_heads, head_dim
        self.eps = eps
        self.dtype = dtype
        self.rnd = rounder(dtype)
        self.cos, self.sin = rope_tables(head_dim, rope_theta, max_positions, 1, dtype)
        self.gate = "model.lookahead_exit_gate" if gate == "lookahead" else "model.early_exit_gate"
        self.acc = np.float64 if accumulate == "f64" else np.float32
        self._w64: dict[int, np.ndarray] = {}

    def _p(self, name: str) -> np.ndarray:
        return self.w[name]

    def _mm(self, x: np.ndarray, weight: np.ndarray) -> np.ndarray:
        # fp32 (or fp64) accumulation; the result is rounded to the model dtype.
        if self.acc is np.float32:
            return self.rnd(np.asarray(x, np.float32) @ weight.T)
        wide = self._w64.get(id(weight))
        if wide is None:
            wide = self._w64[id(weight)] = weight.astype(np.float64)
        return self.rnd((np.asarray(x, np.float64) @ wide.T).astype(np.float32))

    def _layer_stack(self, h: np.ndarray, attend) -> np.ndarray:
        """One loop step over all layers; h is the step input (= residual). Returns final-normed hidden."""

        residual = h
        x = rmsnorm(h, self._p("model.layers.0.input_layernorm.weight"), self.eps, self.dtype)
        for l in range(self.L):
            pre = f"model.layers.{l}."
            q = self._mm(x, self._p(pre + "self_attn.q_proj.weight"))
            k = self._mm(x, self._p(pre + "self_attn.k_proj.weight"))
            v = self._mm(x, self._p(pre + "self_attn.v_proj.weight"))
            n = x.shape[0]
            attn = attend(l, q.reshape(n, self.H, self.D), k.reshape(n, self.Hkv, self.D),
                          v.reshape(n, self.Hkv, self.D))
            o = self._mm(attn.reshape(n, self.H * self.D), self._p(pre + "self_attn.o_proj.weight"))
            residual, x = ouro_sandwich(o, residual, self._p(pre + "input_layernorm_2.weight"),
                                        self._p(pre + "post_attention_layernorm.weight"), self.eps, self.dtype)
            gu = np.concatenate([self._mm(x, self._p(pre + "mlp.gate_proj.weight")),
                                 self._mm(x, self._p(pre + "mlp.up_proj.weight"))], axis=-1)
            m = self._mm(silu_mul(gu, self.dtype), self._p(pre + "mlp.down_proj.weight"))
            nxt = f"model.layers.{l + 1}.input_layernorm.weight" if l + 1 < self.L else "model.norm.weight"
            residual, x = ouro_sandwich(m, residual, self._p(pre + "post_attention_layernorm_2.weight"),
                                        self._p(nxt), self.eps, self.dtype)
        return x

    def _attend(self, kv: np.ndarray, layer: int, q: np.ndarray, k: np.ndarray, v: np.ndarray,
                positions: np.ndarray) -> np.ndarray:
        """Rotate, write K/V of ``positions`` into ``kv[layer]``, attend causally."""

        qr = apply_rope(q, self.cos[positions], self.sin[positions], 1, self.dtype)
        kr = apply_rope(k, self.cos[positions], self.sin[positions], 1, self.dtype)
        kv[layer, 0, positions] = kr
        kv[layer, 1, positions] = v
        end = int(positions[-1]) + 1
        keys = kv[layer, 0, :end].astype(np.float64)
        vals = kv[layer, 1, :end].astype(np.float64)
        group = self.H // self.Hkv
        out = np.zeros(qr.shape, dtype=np.float32)
        mask = np.arange(end)[None, :] <= positions[:, None]
        for h in range(self.H):
            s = qr[:, h].astype(np.float64) @ keys[:, h // group].T * self.D ** -0.5
            s = np.where(mask, s, -np.inf)
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[:, h] = (p @ vals[:, h // group]).astype(np.float32)
        return self.rnd(out)

    def _coda(self, hidden: np.ndarray) -> int:
        logits = self._mm(hidden[None, :], self._p("lm_head.weight"))[0]
        return int(np.argmax(logits))

    def logits(self, hidden: np.ndarray) -> np.ndarray:
        return self._mm(hidden[None, :], self._p("lm_head.weight"))[0]

    def forced_logits(self, prompt: list[int], tokens: list[int], *, max_steps: int, exit_depths: list[int],
                      kv_policy: str = "single") -> np.ndarray:
        """[len(tokens), vocab] float64: row j is the oracle's logits for token j when the request
        decodes ``tokens`` (teacher forcing with its replayed exit depths); row 0 comes from the
        full-depth prefill, row j from decode token j's last loop step."""

        trace: list = []
        self.generate(prompt, len(tokens), max_steps=max_steps, kv_policy=kv_policy,
                      exit_depths=exit_depths[: len(tokens) - 1], forced_tokens=tokens, hidden_trace=trace)
        final = {j: h for j, _, h in trace}  # the last loop step of each token
        return np.stack([self.logits(final[j]) for j in range(len(tokens))]).astype(np.float64)


    def prefill_hidden(self, prompt: list[int], kv: np.ndarray, *, steps: int, slot_of) -> np.ndarray:
        h = self.rnd(self._p("model.embed_tokens.weight")[np.asarray(prompt)])
        pos = np.arange(len(prompt))
        for ut in range(steps):
            base = slot_of(ut) * self.L
            h = self._layer_stack(h, lambda l, q, k, v, base=base: self._attend(kv, base + l, q, k, v, pos))
        return h

    def generate(self, prompt: list[int], max_new_tokens: int, *, max_steps: int, kv_policy: str = "single",
                 exit_depths: list[int] | None = None, threshold: float | None = None, min_steps: int = 1,
                 delayed: bool = False, eos_token_id: int | None = None, forced_tokens: list[int] | None = None,
                 hidden_trace: list | None = None) -> OracleOutput:
        """Greedy CDB decode of one request. ``forced_tokens`` feeds the given tokens back instead
        of the oracle's own (teacher forcing; ``tokens`` still records the oracle's argmax), and
        ``hidden_trace`` collects (token index, loop step, hidden after the step): index 0 is the
        prompt's last position after the full-depth prefill, index j >= 1 the j-th decode token."""

        slots = {"single": 1, "depth_indexed": max_steps, "last_exited": max_steps}[kv_policy]

        def slot_of(step: int) -> int:
            return 0 if kv_policy == "single" else step

        total = len(prompt) + max_new_tokens + 1
        kv = np.zeros((slots * self.L, 2, total, self.Hkv, self.D), dtype=np.float32)
        h = self.prefill_hidden(prompt, kv, steps=max_steps, slot_of=slot_of)
        token = self._coda(h[-1])
        out = OracleOutput(tokens=[token])
        if hidden_trace is not None:
            hidden_trace.append((0, max_steps - 1, h[-1].copy()))
        if forced_tokens is not None:
            token = forced_tokens[0]
        pos = len(prompt)
        gate_w = self._p(self.gate + ".weight").reshape(-1)
        gate_b = float(self._p(self.gate + ".bias").reshape(-1)[0])
        while len(out.tokens) < max_new_tokens and token != eos_token_id:
            k_idx = len(out.tokens) - 1
            depth = None if exit_depths is None else exit_depths[k_idx]
            h = self.rnd(self._p("model.embed_tokens.weight")[[token]])
            cdf, surv = 0.0, 1.0
            pending: float | None = None
            exit_step = max_steps - 1
            for step in range(max_steps):
                base = slot_of(step) * self.L
                h = self._layer_stack(h, lambda l, q, k, v, base=base: self._attend(kv, base + l, q, k, v,
                                                                                   np.array([pos])))
                if hidden_trace is not None:
                    hidden_trace.append((k_idx + 1, step, h[0].copy()))
                if step == max_steps - 1:
                    break
                if depth is not None:
                    if (not delayed and step >= depth) or (delayed and step >= 1 and step - 1 >= depth):
                        exit_step = step
                        break
                    continue
                if threshold is None:
                    continue
                signal = float(gate_logits(h, gate_w, gate_b, self.dtype)[0])
                consumed, source = (signal, step) if not delayed else (pending, step - 1)
                pending = signal
                if consumed is None:
                    continue
                hazard = sigmoid_f32(consumed)
                if not delayed:
                    hazard = float(self.rnd(np.array([hazard], np.float32))[0])
                cdf += hazard * surv
                surv *= 1.0 - hazard
                if source + 1 >= min_steps and cdf >= threshold:
                    exit_step = step
                    break
            out.exit_depths.append(exit_step)
            if kv_policy == "last_exited" and exit_step < max_steps - 1:
                for s in range(exit_step + 1, max_steps):
                    for l in range(self.L):
                        kv[s * self.L + l, :, pos] = kv[exit_step * self.L + l, :, pos]
                out.exit_copies += 1
            token = self._coda(h[0])
            out.tokens.append(token)
            if forced_tokens is not None:
                token = forced_tokens[len(out.tokens) - 1]
            pos += 1
        return out


def forced_choice_stats(ref_logits: np.ndarray, chosen: list[int]) -> dict:
    """How ``chosen`` tokens sit against teacher-forced reference logits: the fraction that are the
    reference's argmax, and the margin (reference max logit minus the reference logit of the
    chosen token; 0 for the argmax) at its worst and on average."""

    idx = np.arange(len(chosen))
    margins = ref_logits.max(axis=1) - ref_logits[idx, np.asarray(chosen)]
    return {"argmax_agreement": float(np.mean(ref_logits.argmax(axis=1) == np.asarray(chosen))),
            "max_logit_margin": float(margins.max()), "mean_logit_margin": float(margins.mean())}
