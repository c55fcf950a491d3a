"""Pin the Ouro oracle before trusting it as the engine's checker."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle.ouro_model import OuroOracle
from tests.ouro_helpers import TINY, tiny_weights


def torch_ouro_forward(w: dict[str, np.ndarray], tokens: list[int], steps: int) -> np.ndarray:
    """Independent fp64 torch forward of the full-depth model over a whole sequence
    (ouro/modeling_ouro.py:377-503, 560-573, 698-709): returns last-position logits."""

    t = {k: torch.from_numpy(v).double() for k, v in w.items()}
    L, H, D, eps = TINY["num_layers"], TINY["num_heads"], TINY["head_dim"], TINY["eps"]
    n = len(tokens)
    inv = 1.0 / (TINY["rope_theta"] ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    freqs = torch.arange(n, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos(), emb.sin()

    def norm(x, name):
        return t[name] * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))

    def rope(x):  # x [H, n, D]
        rot = torch.cat([-x[..., D // 2:], x[..., : D // 2]], dim=-1)
        return x * cos + rot * sin

    h = t["model.embed_tokens.weight"][tokens]
    for _ in range(steps):
        for l in range(L):
            p = f"model.layers.{l}."
            res = h
            x = norm(h, p + "input_layernorm.weight")
            q = (x @ t[p + "self_attn.q_proj.weight"].T).view(n, H, D).transpose(0, 1)
            k = (x @ t[p + "self_attn.k_proj.weight"].T).view(n, H, D).transpose(0, 1)
            v = (x @ t[p + "self_attn.v_proj.weight"].T).view(n, H, D).transpose(0, 1)
            a = F.scaled_dot_product_attention(rope(q), rope(k), v, is_causal=True)
            o = a.transpose(0, 1).reshape(n, H * D) @ t[p + "self_attn.o_proj.weight"].T
            h = res + norm(o, p + "input_layernorm_2.weight")
            res = h
            x = norm(h, p + "post_attention_layernorm.weight")
            m = (F.silu(x @ t[p + "mlp.gate_proj.weight"].T) * (x @ t[p + "mlp.up_proj.weight"].T)) \
                @ t[p + "mlp.down_proj.weight"].T
            h = res + norm(m, p + "post_attention_layernorm_2.weight")
        h = norm(h, "model.norm.weight")
    return (h[-1] @ t["lm_head.weight"].T).numpy()


def make_oracle(w):
    return OuroOracle(w, num_layers=TINY["num_layers"], num_heads=TINY["num_heads"],
                      num_kv_heads=TINY["num_heads"], head_dim=TINY["head_dim"], rope_theta=TINY["rope_theta"],
                      eps=TINY["eps"], dtype="f32", max_positions=256)


def test_oracle_prefill_matches_torch_forward() -> None:
    w = tiny_weights(seed=0)
    oracle = make_oracle(w)
    prompt = list(np.random.default_rng(1).integers(0, TINY["vocab"], 23))
    kv = np.zeros((TINY["num_layers"], 2, 64, TINY["num_heads"], TINY["head_dim"]), np.float32)
    h = oracle.prefill_hidden(prompt, kv, steps=TINY["steps"], slot_of=lambda s: 0)
    np.testing.assert_allclose(oracle.logits(h[-1]), torch_ouro_forward(w, prompt, TINY["steps"]), atol=2e-4)


def test_staged_decode_equals_monolithic_forward() -> None:
    """Prefill prompt[:-1] at full depth, then decode the last token through every
    loop step with depth-indexed KV: the logits equal the monolithic forward over
    the whole prompt (the reference's staged-vs-monolithic property)."""

    w = tiny_weights(seed=2)
    oracle = make_oracle(w)
    prompt = list(np.random.default_rng(3).integers(0, TINY["vocab"], 17))
    steps = TINY["steps"]
    out = oracle.generate(prompt[:-1], 2, max_steps=steps, kv_policy="depth_indexed",
                          exit_depths=[steps - 1])
    want_first = int(np.argmax(torch_ouro_forward(w, prompt[:-1], steps)))
    assert out.tokens[0] == want_first
    # Re-run with the true last prompt token fed as the decode token.
    kv = np.zeros((steps * TINY["num_layers"], 2, 64, TINY["num_heads"], TINY["head_dim"]), np.float32)
    oracle.prefill_hidden(prompt[:-1], kv, steps=steps, slot_of=lambda s: s)
    h = oracle.rnd(oracle.w["model.embed_tokens.weight"][[prompt[-1]]])
    pos = np.array([len(prompt) - 1])
    for s in range(steps):
        h = oracle._layer_stack(h, lambda l, q, k, v, s=s: oracle._attend(kv, s * TINY["num_layers"] + l, q, k, v,
                                                                          pos))
    np.testing.assert_allclose(oracle.logits(h[0]), torch_ouro_forward(w, prompt, steps), atol=2e-4)


def test_replayed_depths_are_recorded_and_single_slot_decodes() -> None:
    w = tiny_weights(seed=4)
    oracle = make_oracle(w)
    depths = [0, 3, 1, 2, 0]
    out = oracle.generate([5, 6, 7, 8], 6, max_steps=4, kv_policy="single", exit_depths=depths)
    assert out.exit_depths == depths and len(out.tokens) == 6
    torch.manual_seed(0)


def test_forced_logits_pin_the_parity_statistics() -> None:
    """Teacher forcing with the oracle's own greedy tokens: every row's argmax is the token that
    follows (agreement 1, margins 0), and row 0 equals the independent torch forward's last
    position. A planted wrong token at one step shows up as that step's margin and as one
    disagreement."""

    from oracle.ouro_model import forced_choice_stats

    w = tiny_weights(seed=3, std=0.05)
    oracle = make_oracle(w)
    prompt = list(range(100, 112))
    depths = [3, 1, 0, 2, 3]
    out = oracle.generate(prompt, 6, max_steps=4, kv_policy="single", exit_depths=depths)
    logits = oracle.forced_logits(prompt, out.tokens, max_steps=4, exit_depths=depths)
    assert logits.shape == (6, TINY["vocab"])
    np.testing.assert_allclose(logits[0], torch_ouro_forward(w, prompt, 4), rtol=1e-4, atol=1e-4)
    stats = forced_choice_stats(logits, out.tokens)
    assert stats == {"argmax_agreement": 1.0, "max_logit_margin": 0.0, "mean_logit_margin": 0.0}
    wrong = list(out.tokens)
    wrong[2] = int(np.argsort(logits[2])[-2])  # the runner-up at step 2
    stats = forced_choice_stats(logits, wrong)
    assert stats["argmax_agreement"] == 5 / 6
    assert stats["max_logit_margin"] == float(logits[2].max() - logits[2][wrong[2]]) > 0
