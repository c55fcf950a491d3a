"""Pin the Huginn oracle before trusting it as the engine's checker."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from tests.huginn_helpers import TINY_HUGINN, make_huginn_oracle, tiny_huginn_weights

T = TINY_HUGINN


def torch_huginn_forward(w: dict[str, np.ndarray], tokens: list[int], steps: int) -> np.ndarray:
    """Independent float64 torch forward over a whole sequence at fixed depth
    (huginn/modeling_huginn.py:141-338, 399-505): rotary pairs as complex products,
    attention from scaled_dot_product_attention; returns last-position logits."""

    t = {k: torch.from_numpy(v).double() for k, v in w.items()}
    E, H, eps = T["n_embd"], T["n_heads"], T["eps"]
    D = E // H
    n = len(tokens)
    inv = 1.0 / (T["rope_base"] ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    rot = torch.polar(torch.ones(n, D // 2, dtype=torch.float64),
                      torch.arange(n, dtype=torch.float64)[:, None] * inv[None, :])

    def norm(x, name):
        return t[name] * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))

    def rope(x):  # [n, H, D]: rotate (even, odd) pairs by e^{i * angle}
        c = torch.view_as_complex(x.reshape(n, H, D // 2, 2).contiguous())
        return torch.view_as_real(c * rot[:, None, :]).reshape(n, H, D)

    def block(p, x):
        qkv = norm(x, p + "norm_1.weight") @ t[p + "attn.Wqkv.weight"].T
        q, k, v = qkv[:, :E].view(n, H, D), qkv[:, E:2 * E].view(n, H, D), qkv[:, 2 * E:].view(n, H, D)
        q = rope(q + t[p + "attn.qk_bias"][0, 0])
        k = rope(k + t[p + "attn.qk_bias"][1, 0])
        a = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), is_causal=True)
        x = norm(a.transpose(0, 1).reshape(n, E) @ t[p + "attn.proj.weight"].T + x, p + "norm_2.weight")
        gu = norm(x, p + "norm_3.weight") @ t[p + "mlp.fc.weight"].T
        g, u = gu.chunk(2, dim=-1)
        return norm((F.silu(g) * u) @ t[p + "mlp.proj.weight"].T + x, p + "norm_4.weight")

    x = t["transformer.wte.weight"][tokens] * E ** 0.5
    for i in range(T["n_prelude"]):
        x = block(f"transformer.prelude.{i}.", x)
    inj, state = x, torch.zeros_like(x)
    for _ in range(steps):
        state = torch.cat([state, inj], dim=-1) @ t["transformer.adapter.weight"].T
        for i in range(T["n_core"]):
            state = block(f"transformer.core_block.{i}.", state)
    x = norm(state, "transformer.ln_f.weight")
    for i in range(T["n_coda"]):
        x = block(f"transformer.coda.{i}.", x)
    x = norm(x, "transformer.ln_f.weight")
    return (x[-1] @ t["lm_head.weight"].T).numpy()


def test_lm_head_is_tied_to_the_embedding() -> None:
    w = tiny_huginn_weights(seed=0)
    np.testing.assert_array_equal(w["lm_head.weight"], w["transformer.wte.weight"])


def test_oracle_prefill_matches_torch_forward() -> None:
    w = tiny_huginn_weights(seed=0)
    oracle = make_huginn_oracle(w)
    prompt = list(np.random.default_rng(1).integers(0, T["vocab"], 21))
    kv = np.zeros((oracle.num_cache_layers(1), 2, 64, T["n_heads"], T["n_embd"] // T["n_heads"]), np.float32)
    h = oracle.prefill_hidden(prompt, kv, steps=T["steps"], slot_of=lambda s: 0, num_slots=1)
    np.testing.assert_allclose(oracle.logits(h[-1]), torch_huginn_forward(w, prompt, T["steps"]), atol=2e-4)


def test_staged_decode_equals_monolithic_forward() -> None:
    """Full-depth prefill of prompt[:-1], then the last prompt token through the prelude,
    every core step (depth-indexed slots) and the coda at its position: the logits equal
    the monolithic forward over the whole prompt."""

    w = tiny_huginn_weights(seed=2)
    oracle = make_huginn_oracle(w)
    prompt = list(np.random.default_rng(3).integers(0, T["vocab"], 15))
    steps = T["steps"]
    kv = np.zeros((oracle.num_cache_layers(steps), 2, 64, T["n_heads"], T["n_embd"] // T["n_heads"]), np.float32)
    oracle.prefill_hidden(prompt[:-1], kv, steps=steps, slot_of=lambda s: s, num_slots=steps)
    p = np.array([len(prompt) - 1])
    inj = oracle.prelude([prompt[-1]], kv, p)
    state = np.zeros_like(inj)
    for s in range(steps):
        state = oracle.core_step(state, inj, kv, s, p)
    h = oracle.coda(state, kv, steps, p)
    np.testing.assert_allclose(oracle.logits(h[0]), torch_huginn_forward(w, prompt, steps), atol=2e-4)


def test_generate_first_token_is_the_monolithic_argmax_and_replay_is_recorded() -> None:
    w = tiny_huginn_weights(seed=4)
    oracle = make_huginn_oracle(w)
    prompt = [5, 9, 200, 31, 7]
    depths = [0, 3, 1, 2]
    out = oracle.generate(prompt, 5, max_steps=T["steps"], kv_policy="single", exit_depths=depths)
    assert out.tokens[0] == int(np.argmax(torch_huginn_forward(w, prompt, T["steps"])))
    assert out.exit_depths == depths and len(out.tokens) == 5


def test_latent_difference_closed_forms() -> None:
    oracle = make_huginn_oracle(tiny_huginn_weights(seed=0))
    s = np.random.default_rng(0).standard_normal(T["n_embd"]).astype(np.float32)
    assert oracle.latent_diff(s, s) == 0.0
    assert abs(oracle.latent_diff(4 * s, s) - 0.75) < 1e-6
    assert oracle.latent_diff(s, np.zeros_like(s)) == 1.0
