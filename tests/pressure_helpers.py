"""Shared pieces of the KV-pressure tests: an over-subscribed workload and the soft-reset oracle."""

from __future__ import annotations

import numpy as np


def pressure_workload(seed: int = 5, n: int = 8, new_tokens: int = 32, vocab: int = 49152):
    """8 prompts of 16-64 tokens, 32 new tokens each, and a replayed exit depth per decode token."""

    rng = np.random.default_rng(seed)
    lengths = rng.integers(16, 65, n)
    prompts = [rng.integers(0, vocab, int(length)).tolist() for length in lengths]
    depth_rng = np.random.default_rng(seed + 1)
    depths = [depth_rng.choice(4, size=new_tokens - 1, p=[0.15, 0.25, 0.3, 0.3]).tolist() for _ in range(n)]
    return prompts, [new_tokens] * n, depths


# 30 blocks of 4 tokens for 8 requests that grow to 12-24 blocks each.
PRESSURE = dict(num_blocks=30, block_size=4, max_model_len=512, max_num_batched_tokens=512, max_num_seqs=16,
                safety_margin=0.0, synthetic_exit_replay=True, delay_gate_consumption=False)


def preemption_cuts(recompute_events, prompts: list[list[int]]) -> dict[int, list[int]]:
    """Generated-token count of each soft reset, per request index, in order."""

    cuts: dict[int, list[int]] = {}
    for _, request_id, length in recompute_events:
        index = int(request_id.split("-")[1])
        cuts.setdefault(index, []).append(length - len(prompts[index]))
    return cuts


def composed_oracle(oracle_run, prompt: list[int], mnt: int, depths: list[int], cuts: list[int]):
    """Tokens and exit depths of a request soft-reset after ``cuts[i]`` generated tokens.

    Each segment re-prefills prompt + the tokens so far at full depth; its first token is the
    prefill's, and the pending token's replayed depth is dropped (cdb/requests.py:111-126).
    ``oracle_run(prompt, new_tokens, depths)`` returns an object with ``tokens`` and
    ``exit_depths`` (one per decode token)."""

    tokens: list[int] = []
    exits: list[int] = []
    for cut in [*cuts, mnt]:
        seg = oracle_run(prompt + tokens, mnt - len(tokens), depths[len(tokens):])
        take = cut - len(tokens)
        exits += seg.exit_depths[: take - 1] if cut < mnt else seg.exit_depths
        tokens += seg.tokens[:take]
    return tokens, exits
