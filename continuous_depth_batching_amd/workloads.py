"""Seeded synthetic workloads for the CDB decode step.

* ``decode_attention_microbench``: the kernel-only mixed-depth paged decode
  attention case -- bf16 q [B, H, D]; KV pages of 16 tokens in a pool holding
  every row's pages in each of ``num_slots`` loop-slot cache layers; per-row
  context lengths uniform in [ctx_min, ctx_max]; per-row loop step uniform in
  {0..num_slots-1}; block tables drawn from a seeded random permutation of the
  page pool; K/V values N(0, 1).
* ``lognormal_requests`` / ``categorical_exit_trace`` / ``poisson_exit_trace``:
  request length distributions and per-token replayed exit depths for the
  end-to-end engine runs. Exit traces are 0-based recurrent steps, one per
  staged decode token (``max_new_tokens - 1`` entries per request), the
  format ``generate_batch(exit_depths=...)`` takes
  (continuous_depth_batching/continuous_api.py:395-399).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class DecodeAttentionCase:
    q: torch.Tensor            # [B, H, D]
    k_new: torch.Tensor        # [B, Hkv, D]
    v_new: torch.Tensor
    kv_pool: torch.Tensor      # [slots, 2, rows, Hkv, D]
    slot_offset: torch.Tensor  # [B] int32 cache-layer offset (the row's loop slot)
    block_table: torch.Tensor  # [B, W] int32
    seqlens: torch.Tensor      # [B] int32 position of the new token
    rope_cos: torch.Tensor     # [max_pos, D/2] float32
    rope_sin: torch.Tensor
    block_size: int
    contexts: np.ndarray       # [B] tokens attended per row (position + 1)

    def algorithmic_bytes(self) -> int:
        """HBM bytes one launch must move: K/V of every attended token, q, out,
        the appended K/V, block-table entries and positions."""

        num_rows, num_heads, head_dim = self.q.shape
        num_kv_heads = self.k_new.shape[1]
        elem = self.q.element_size()
        kv = int(self.contexts.sum()) * num_kv_heads * head_dim * elem * 2
        q_out = 2 * num_rows * num_heads * head_dim * elem
        appended = 2 * num_rows * num_kv_heads * head_dim * elem
        tables = int(((self.contexts + self.block_size - 1) // self.block_size).sum()) * 4
        return kv + q_out + appended + tables + 4 * num_rows


def rope_tables_torch(head_dim: int, theta: float, max_positions: int, dtype: torch.dtype,
                      device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """Split-half RoPE tables as the reference's rotary module builds them
    (ouro/modeling_ouro.py:544-573): fp32 angles, cos/sin cast to the model dtype,
    returned as fp32 [max_positions, D/2]."""

    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(device=device,
                                                                                  dtype=torch.float) / head_dim))
    positions = torch.arange(max_positions, device=device, dtype=torch.float32)
    freqs = positions[:, None] * inv_freq[None, :]
    return freqs.cos().to(dtype).float().contiguous(), freqs.sin().to(dtype).float().contiguous()


def decode_attention_microbench(
    *,
    num_rows: int = 1024,
    num_heads: int = 16,
    head_dim: int = 128,
    ctx_min: int = 128,
    ctx_max: int = 8192,
    num_slots: int = 4,
    block_size: int = 16,
    seed: int = 0,
    dtype: torch.dtype = torch.bfloat16,
    device: torch.device | str = "cuda",
) -> DecodeAttentionCase:
    device = torch.device(device)
    rng = np.random.default_rng(seed)
    contexts = rng.integers(ctx_min, ctx_max + 1, size=num_rows).astype(np.int64)
    slots = rng.integers(0, num_slots, size=num_rows).astype(np.int32)
    pages = (contexts + block_size - 1) // block_size
    total_pages = int(pages.sum())
    perm = rng.permutation(total_pages).astype(np.int32)
    width = int(pages.max())
    table = np.full((num_rows, width), -1, dtype=np.int32)
    offsets = np.concatenate([[0], np.cumsum(pages)])
    for b in range(num_rows):
        table[b, : pages[b]] = perm[offsets[b]: offsets[b + 1]]
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    rows = total_pages * block_size
    pool = torch.empty((num_slots, 2, rows, num_heads, head_dim), dtype=dtype, device=device)
    for s in range(num_slots):
        for kv in range(2):
            pool[s, kv].normal_(generator=gen)
    q = torch.randn((num_rows, num_heads, head_dim), generator=gen, device=device).to(dtype)
    k_new = torch.randn((num_rows, num_heads, head_dim), generator=gen, device=device).to(dtype)
    v_new = torch.randn((num_rows, num_heads, head_dim), generator=gen, device=device).to(dtype)
    cos, sin = rope_tables_torch(head_dim, 10000.0, int(contexts.max()), dtype, device)
    return DecodeAttentionCase(
        q=q, k_new=k_new, v_new=v_new, kv_pool=pool,
        slot_offset=torch.from_numpy(slots).to(device),
        block_table=torch.from_numpy(table).to(device),
        seqlens=torch.from_numpy((contexts - 1).astype(np.int32)).to(device),
        rope_cos=cos, rope_sin=sin, block_size=block_size, contexts=contexts,
    )


@dataclass
class PrefillAttentionCase:
    """A fresh-prompt prefill batch: every sequence attends causally over its own prompt."""

    q: torch.Tensor            # [T, H, D] rotated queries
    kv_pool: torch.Tensor      # [1, 2, rows, Hkv, D]
    block_table: torch.Tensor  # [S, W] int32
    table_row: torch.Tensor    # [S] int32
    cu_q: torch.Tensor         # [S+1] int32
    past: torch.Tensor         # [S] int32 (zeros: fresh prompts)
    tile_seq: torch.Tensor
    tile_q0: torch.Tensor
    lens: np.ndarray
    block_size: int
    past_lens: np.ndarray | None = None

    def flops(self) -> int:
        """4 * H * D * causal (query, key) pairs: QK^T and PV, 2 flops per multiply-add."""

        _, h, d = self.q.shape
        past = np.zeros_like(self.lens) if self.past_lens is None else self.past_lens
        pairs = int((self.lens * past + self.lens * (self.lens + 1) // 2).sum())
        return 4 * h * d * pairs


def prefill_attention_batch(*, lens: np.ndarray, num_heads: int = 16, head_dim: int = 128, block_size: int = 16,
                            seed: int = 0, dtype: torch.dtype = torch.bfloat16, past: np.ndarray | None = None,
                            device: torch.device | str = "cuda") -> PrefillAttentionCase:
    """A prefill batch: sequence s has `past[s]` cached positions (zero: fresh prompts) and
    `lens[s]` new query tokens; the pool holds random K/V for every position."""

    from . import ops

    device = torch.device(device)
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    past_arr = np.zeros_like(lens) if past is None else np.asarray(past, dtype=np.int64)
    pages = (past_arr + lens + block_size - 1) // block_size
    perm = rng.permutation(int(pages.sum())).astype(np.int32)
    table = np.full((lens.size, int(pages.max())), -1, dtype=np.int32)
    off = np.concatenate([[0], np.cumsum(pages)])
    for s in range(lens.size):
        table[s, : pages[s]] = perm[off[s]: off[s + 1]]
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    pool = torch.empty((1, 2, int(pages.sum()) * block_size, num_heads, head_dim), dtype=dtype, device=device)
    pool.normal_(generator=gen)
    q = torch.randn((int(lens.sum()), num_heads, head_dim), generator=gen, device=device).to(dtype)
    tile_seq, tile_q0 = ops.prefill_tiles(lens, past_arr)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).to(device)
    return PrefillAttentionCase(q=q, kv_pool=pool, block_table=i32(table), table_row=i32(np.arange(lens.size)),
                                cu_q=i32(np.concatenate([[0], np.cumsum(lens)])), past=i32(past_arr),
                                tile_seq=i32(tile_seq), tile_q0=i32(tile_q0), lens=lens, block_size=block_size,
                                past_lens=past_arr)


def lognormal_lengths(rng: np.random.Generator, n: int, mu: float, sigma: float, lo: int, hi: int) -> np.ndarray:
    return np.clip(np.rint(rng.lognormal(mu, sigma, size=n)), lo, hi).astype(np.int64)


def lognormal_requests(*, num_requests: int, vocab_size: int, prompt_mu: float, prompt_sigma: float,
                       prompt_range: tuple[int, int], output_mu: float, output_sigma: float,
                       output_range: tuple[int, int], seed: int) -> tuple[list[list[int]], list[int]]:
    """Prompts with uniform token ids and lognormal lengths, and lognormal output lengths."""

    rng = np.random.default_rng(seed)
    prompt_lens = lognormal_lengths(rng, num_requests, prompt_mu, prompt_sigma, *prompt_range)
    output_lens = lognormal_lengths(rng, num_requests, output_mu, output_sigma, *output_range)
    prompts = [rng.integers(0, vocab_size, size=int(n)).tolist() for n in prompt_lens]
    return prompts, [int(n) for n in output_lens]


def categorical_exit_trace(max_new_tokens: list[int], probabilities: tuple[float, ...], seed: int) -> list[list[int]]:
    """0-based exit steps drawn from a categorical over depths 1..len(probabilities)."""

    rng = np.random.default_rng(seed)
    p = np.asarray(probabilities, dtype=np.float64)
    p = p / p.sum()
    return [rng.choice(len(p), size=max(0, n - 1), p=p).astype(int).tolist() for n in max_new_tokens]


def poisson_exit_trace(max_new_tokens: list[int], mean: float, max_steps: int, seed: int) -> list[list[int]]:
    """0-based exit steps from Poisson(mean) depths truncated to [1, max_steps]."""

    rng = np.random.default_rng(seed)
    return [(np.clip(rng.poisson(mean, size=max(0, n - 1)), 1, max_steps) - 1).astype(int).tolist()
            for n in max_new_tokens]


# The headline decode workload: 256 sequences at the Ouro-1.4B shape, prompts lognormal(5.5, 1.0)
# clipped to [8, 2048], outputs lognormal(5.0, 0.8) clipped to [16, 1024], uniform token ids, and
# 1-indexed exit depths drawn from the categorical {1: .15, 2: .25, 3: .30, 4: .30}.
OURO_EXIT_PROBS = (0.15, 0.25, 0.30, 0.30)


def ouro_decode_workload(num_seqs: int = 256, vocab_size: int = 49152) -> tuple[list[list[int]], list[int],
                                                                                 list[list[int]]]:
    """(prompts, max_new_tokens, 0-based exit depths) of the seeded headline decode workload."""

    prompts, outputs = lognormal_requests(num_requests=num_seqs, vocab_size=vocab_size, prompt_mu=5.5,
                                          prompt_sigma=1.0, prompt_range=(8, 2048), output_mu=5.0,
                                          output_sigma=0.8, output_range=(16, 1024), seed=1)
    return prompts, outputs, categorical_exit_trace(outputs, OURO_EXIT_PROBS, seed=2)


def huginn_decode_workload(num_seqs: int = 128, new_tokens: int = 256,
                           vocab_size: int = 65536) -> tuple[list[list[int]], list[int], list[list[int]]]:
    """(prompts, max_new_tokens, 0-based exit steps) of the seeded Huginn-0125 decode workload:
    prompts lognormal(5.0, 0.9) clipped to [8, 1024] with uniform ids, `new_tokens` new tokens
    each, and per-token exit steps from Poisson(12) truncated to [1, 32]."""

    prompts, _ = lognormal_requests(num_requests=num_seqs, vocab_size=vocab_size, prompt_mu=5.0, prompt_sigma=0.9,
                                    prompt_range=(8, 1024), output_mu=5.0, output_sigma=0.8,
                                    output_range=(16, 1024), seed=3)
    outputs = [new_tokens] * num_seqs
    return prompts, outputs, poisson_exit_trace(outputs, mean=12.0, max_steps=32, seed=4)
