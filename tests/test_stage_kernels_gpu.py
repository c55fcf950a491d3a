"""HIP stage kernels vs the oracle (through the C ABI).

Integer/index work (row copies, argmax, exit decisions, exit-KV copies,
prefill KV writes) must be bit-exact. Floating-point rows: RMSNorm/SiLU may
differ from the oracle by the accumulation order of the mean of squares, so
they are compared with the bf16 tolerance (max 2e-2, mean 2e-3) and must agree
exactly on at least 99% of elements; prefill attention uses the decode
attention tolerance (max 2e-2 / mean 2e-3 for bf16, 2e-5 / 2e-6 for fp32).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import stage
from oracle.bf16 import rounder
from oracle.paged_attention import apply_rope, prefill_attention, rope_tables, write_rows

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f32": torch.float32}


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("width", [256, 2048, 5280])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_rmsnorm_fused(dtype: str, width: int, mode: int) -> None:
    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(width + mode)
    rnd = rounder(dtype)
    x, r = rnd(rng.standard_normal((2, 37, width)).astype(np.float32))
    wa, wb = rnd(1.0 + 0.1 * rng.standard_normal((2, width)).astype(np.float32))
    xt, rt = dev(x, DT[dtype]), dev(r, DT[dtype])
    h = torch.empty_like(xt)
    y = torch.empty_like(xt)
    ops.rmsnorm_fused_raw(xt, rt if mode else None, dev(wa, DT[dtype]), dev(wb, DT[dtype]) if mode else None, h,
                          y if mode else None, mode, 1e-6, 1e-6)
    if mode == 0:
        want_h, want_y = stage.rmsnorm(x, wa, 1e-6, dtype), None
    elif mode == 1:
        want_h, want_y = stage.ouro_sandwich(x, r, wa, wb, 1e-6, dtype)
    else:
        want_h, want_y = stage.huginn_sandwich(x, r, wa, wb, 1e-6, dtype)
    for got, want in ((host(h), want_h), (host(y) if mode else None, want_y)):
        if want is None:
            continue
        err = np.abs(got - want)
        assert err.max() <= (2e-2 if dtype == "bf16" else 1e-5) * max(1.0, np.abs(want).max())
        assert np.mean(got == want) >= 0.99 if dtype == "bf16" else True


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_silu_mul(dtype: str) -> None:
    from continuous_depth_batching_amd import ops

    gu = rounder(dtype)(np.random.default_rng(0).standard_normal((33, 2 * 5632)).astype(np.float32) * 3)
    out = torch.ops.cdb.silu_mul(dev(gu, DT[dtype]))
    want = stage.silu_mul(gu, dtype)
    got = host(out)
    assert np.abs(got - want).max() <= (2e-2 if dtype == "bf16" else 1e-5) * np.abs(want).max()
    if dtype == "bf16":
        assert np.mean(got == want) >= 0.99


def test_silu_mul_bf16_is_torch_silu_on_every_input() -> None:
    """The bf16 SiLU (hardware exponential, IEEE division) on all 65536 bf16 bit
    patterns, each times an up value of 1: the same bits as torch's own bf16 SiLU for
    every input, NaN where torch gives NaN (the NaN inputs, and -inf: -inf / inf)."""

    g = torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16))
    g = g.view(torch.bfloat16).reshape(64, 1024).cuda()
    out = torch.ops.cdb.silu_mul(torch.cat([g, torch.ones_like(g)], dim=1))
    want = torch.nn.functional.silu(g)
    torch.cuda.synchronize()
    same = out.view(torch.int16) == want.view(torch.int16)
    nan = torch.isnan(out) & torch.isnan(want)
    assert bool((same | nan).all()), f"{int((~(same | nan)).sum())} inputs differ"
    assert bool((torch.isnan(out) == torch.isnan(want)).all())
    assert int(torch.isnan(out).sum()) == 254 + 1


def test_copy_rows_gather_scatter_and_token_gather() -> None:
    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(1)
    bank = torch.from_numpy(rng.standard_normal((40, 2048)).astype(np.float32)).cuda().bfloat16()
    idx = torch.tensor([3, 0, 39, -1, 7], dtype=torch.int64, device="cuda")
    got = torch.ops.cdb.gather_rows(bank, idx)
    want = bank[idx.clamp(min=0)].clone()
    want[3] = 0
    assert torch.equal(got, want)
    dst = bank.clone()
    torch.ops.cdb.scatter_rows_(dst, torch.tensor([5, -1, 9], dtype=torch.int64, device="cuda"), got[:3])
    ref = bank.clone()
    ref[5] = got[0]
    ref[9] = got[2]
    assert torch.equal(dst, ref)
    tokens = torch.arange(100, 110, dtype=torch.int64, device="cuda").view(10, 1)
    gathered = torch.empty((4, 1), dtype=torch.int64, device="cuda")
    ops.copy_rows_raw(tokens, torch.tensor([9, 0, 4, 4], dtype=torch.int64, device="cuda"), gathered, None, 4)
    assert gathered.view(-1).tolist() == [109, 100, 104, 104]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_argmax_first_max_bit_exact(dtype: str) -> None:
    rng = np.random.default_rng(2)
    logits = rounder(dtype)(rng.standard_normal((65, 49152)).astype(np.float32))
    logits[3, [10, 20000, 49151]] = 50.0  # ties: first wins
    logits[4, [7, 30000]] = np.nan  # a NaN counts as the maximum, first one wins
    logits[5, :] = -np.inf
    got = torch.ops.cdb.argmax(dev(logits, DT[dtype])).cpu().numpy()
    np.testing.assert_array_equal(got, stage.argmax(logits))
    np.testing.assert_array_equal(got, torch.from_numpy(logits).argmax(-1).numpy())


@pytest.mark.parametrize("vocab", [1001, 8, 65536 + 5])
def test_argmax_unaligned_and_tail_vocab(vocab: int) -> None:
    rng = np.random.default_rng(vocab)
    logits = rounder("bf16")(rng.standard_normal((9, vocab)).astype(np.float32))
    logits[0, vocab - 1] = 99.0  # the maximum in the scalar tail
    got = torch.ops.cdb.argmax(dev(logits, DT["bf16"])).cpu().numpy()
    np.testing.assert_array_equal(got, stage.argmax(logits))


@pytest.mark.parametrize("delayed", [False, True])
def test_exit_gate_hazard_decisions_bit_exact(delayed: bool) -> None:
    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(3)
    rows, width, steps_max = 64, 2048, 4
    rnd = rounder("bf16")
    w = rnd(rng.standard_normal(width).astype(np.float32) * 0.02)
    bias = rnd(np.array([0.1], np.float32))
    state = ops.GateState.allocate(128, torch.device("cuda"))
    slots = rng.permutation(128)[:rows].astype(np.int64)
    state.reset(dev(slots))
    policies = [stage.TokenPolicy() for _ in range(rows)]
    pending = [None] * rows
    threshold = 0.6
    for step in range(steps_max):
        h = rnd(rng.standard_normal((rows, width)).astype(np.float32))
        signal = torch.empty(rows, dtype=torch.bfloat16, device="cuda")
        flags = torch.empty(rows, dtype=torch.uint8, device="cuda")
        ops.exit_gate_raw(dev(h, torch.bfloat16), None, dev(w, torch.bfloat16), dev(bias, torch.bfloat16), signal,
                          state, dev(slots), dev(np.full(rows, step, np.int32)), None, flags, rows,
                          kind=ops.GATE_HAZARD, rule=ops.RULE_CUMULATIVE_HAZARD, delayed=delayed,
                          round_hazard=not delayed, min_steps=2, max_steps=steps_max, threshold=threshold)
        sig = host(signal)
        want_sig = stage.gate_logits(h, w, float(bias[0]), "bf16")
        assert np.mean(sig == want_sig) >= 0.98
        got_flags = flags.cpu().numpy().astype(bool)
        for b in range(rows):
            if step == steps_max - 1:
                want = True
            elif delayed:
                want = False
                if pending[b] is not None:
                    want = policies[b].consume(rule="hazard", signal=pending[b], source_step=step - 1,
                                               threshold=threshold, min_steps=2)
            else:
                want = policies[b].consume(rule="hazard", signal=float(sig[b]), source_step=step,
                                           threshold=threshold, min_steps=2, round_hazard="bf16")
            pending[b] = float(sig[b])
            assert got_flags[b] == want, (step, b)
    cdf = state.cdf.cpu().numpy()[slots]
    if not delayed:
        np.testing.assert_array_equal(cdf, [p.exit_cdf for p in policies])


def test_exit_gate_synthetic_replay_and_latent_difference() -> None:
    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(4)
    rows, width = 16, 5280
    h, prev = rounder("bf16")(rng.standard_normal((2, rows, width)).astype(np.float32))
    state = ops.GateState.allocate(rows, torch.device("cuda"))
    idx = dev(np.arange(rows, dtype=np.int64))
    state.reset(idx)
    synth = rng.integers(0, 4, rows).astype(np.int32)
    steps = rng.integers(0, 4, rows).astype(np.int32)
    signal = torch.empty(rows, dtype=torch.bfloat16, device="cuda")
    flags = torch.empty(rows, dtype=torch.uint8, device="cuda")
    ops.exit_gate_raw(dev(h, torch.bfloat16), dev(prev, torch.bfloat16), None, None, signal, state, idx, dev(steps),
                      dev(synth), flags, rows, kind=ops.GATE_LATENT_DIFF, rule=ops.RULE_DIRECT_THRESHOLD,
                      delayed=False, round_hazard=False, min_steps=1, max_steps=4, threshold=None)
    want = [stage.decide_exit(step=int(s), max_steps=4, synthetic_depth=int(d), policy=None, signal=None,
                              rule="direct", threshold=None, min_steps=1) for s, d in zip(steps, synth)]
    assert flags.cpu().numpy().astype(bool).tolist() == want
    want_sig = stage.latent_diff(h, prev, "bf16")
    np.testing.assert_allclose(host(signal), want_sig, rtol=2 ** -7)  # within one bf16 step; pinned exactly below


def test_latent_difference_signal_and_threshold_decisions_are_exact() -> None:
    """Huginn's exit signal R(|R(h - prev)| / |h|) (huginn/exit_gates.py:33-40) and the direct
    threshold rule (signal < threshold, cdb/exit_policy.py:165-169), pinned tighter than a
    tolerance: the signal must equal the oracle's bf16 value exactly on nearly every row (the
    float32 sums differ from the oracle's float64 ones only in order, which can move a value
    across a bf16 rounding boundary) and within one bf16 step on all; and the decision must
    flip exactly at each row's own signal: a threshold equal to the signal keeps the row, the
    next float64 above it lets the row exit."""

    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(14)
    rows, width = 64, 5280
    h = rounder("bf16")(rng.standard_normal((rows, width)).astype(np.float32))
    scales = np.logspace(-3, 0.5, rows).astype(np.float32)[:, None]   # signals over three decades
    prev = rounder("bf16")(h + scales * rng.standard_normal((rows, width)).astype(np.float32))
    state = ops.GateState.allocate(rows, torch.device("cuda"))
    idx = dev(np.arange(rows, dtype=np.int64))
    steps = dev(np.ones(rows, np.int32))
    synth = dev(np.full(rows, -1, np.int32))
    signal = torch.empty(rows, dtype=torch.bfloat16, device="cuda")
    flags = torch.empty(rows, dtype=torch.uint8, device="cuda")
    h_d, prev_d = dev(h, torch.bfloat16), dev(prev, torch.bfloat16)

    def gate(threshold):
        state.reset(idx)
        ops.exit_gate_raw(h_d, prev_d, None, None, signal, state, idx, steps, synth, flags, rows,
                          kind=ops.GATE_LATENT_DIFF, rule=ops.RULE_DIRECT_THRESHOLD, delayed=False,
                          round_hazard=False, min_steps=1, max_steps=4, threshold=threshold)
        torch.cuda.synchronize()
        return host(signal).astype(np.float64), flags.cpu().numpy().astype(bool)

    got, _ = gate(None)
    want = stage.latent_diff(h, prev, "bf16").astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.abs(want))) - 7)
    assert np.all(np.abs(got - want) <= ulp), np.abs(got - want).max()
    assert np.mean(got == want) >= 0.95, np.mean(got == want)
    for b in range(0, rows, 7):
        s = float(got[b])
        _, at = gate(s)
        _, above = gate(float(np.nextafter(s, np.inf)))
        np.testing.assert_array_equal(at, got < s)
        np.testing.assert_array_equal(above, got <= s)
        assert not at[b] and above[b]
        # The engine's decision path on the oracle's own signal agrees wherever the signals agree.
        oracle = np.array([stage.decide_exit(step=1, max_steps=4, synthetic_depth=None, policy=stage.TokenPolicy(),
                                             signal=float(w), rule="direct", threshold=s, min_steps=1) for w in want])
        same = got == want
        np.testing.assert_array_equal(at[same], oracle[same])


def test_table_updates_apply_the_device_count_inside_a_graph() -> None:
    """cdb_table_updates writes table[idx[i]] = val[i] for i < min(count, capacity), with the count
    read on the device: a captured graph applies whatever the buffers hold at replay time.
    Cells outside the table are skipped. Each replay is checked against the host's own copy,
    with eager work and synchronizations between replays."""

    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(9)
    rows, width, capacity = 40, 24, 64
    table = torch.full((rows, width), -1, dtype=torch.int32, device="cuda")
    want = np.full((rows, width), -1, np.int32)
    idx = torch.zeros(capacity, dtype=torch.int64, device="cuda")
    val = torch.zeros(capacity, dtype=torch.int32, device="cuda")
    count = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        ops.table_updates_raw(table, idx, val, count, capacity)   # warm-up with count 0: no change
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ops.table_updates_raw(table, idx, val, count, capacity)
    stream.synchronize()
    assert bool((table == -1).all())
    for replay, n in enumerate((5, 64, 0, 70, 17)):
        cells = rng.choice(rows * width, size=min(n, capacity), replace=False).astype(np.int64)
        values = rng.integers(0, 1 << 20, size=cells.size).astype(np.int32)
        if n >= 17:
            cells[3] = rows * width + 5      # outside the table: skipped
            cells[4] = -2
        idx[:cells.size].copy_(torch.from_numpy(cells))
        val[:values.size].copy_(torch.from_numpy(values))
        count.fill_(n)
        torch.cuda.synchronize()
        print(f"[table updates] replay {replay}: count {n}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        for c, v in zip(cells[:min(n, capacity)], values[:min(n, capacity)]):
            if 0 <= c < rows * width:
                want.reshape(-1)[c] = v
        np.testing.assert_array_equal(table.cpu().numpy(), want)


def test_exit_kv_copy_bit_exact() -> None:
    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(5)
    layers, slots, base = 3, 4, 2
    pool = rng.standard_normal((base + layers * slots + 1, 2, 64, 4, 64)).astype(np.float32)
    rows = np.array([5, 17, 40], np.int64)
    exit_slot = np.array([0, 2, 3], np.int32)
    pt = dev(pool, torch.bfloat16)
    want = host(pt).copy()
    stage.exit_kv_copy(want, rows, exit_slot, layer_base=base, core_layers=layers, num_slots=slots)
    ops.exit_kv_copy_raw(ops.KVPoolView(pt, 16), dev(rows), dev(exit_slot), 3, layer_base=base, core_layers=layers,
                         num_slots=slots)
    np.testing.assert_array_equal(host(pt), want)


@pytest.mark.parametrize("dtype,head_dim,heads,kv_heads", [("bf16", 128, 16, 16), ("f32", 64, 4, 4),
                                                           ("bf16", 96, 6, 3), ("f32", 128, 2, 2)])
def test_rope_kv_write_and_prefill_attention(dtype: str, head_dim: int, heads: int, kv_heads: int) -> None:
    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(head_dim + heads)
    rnd = rounder(dtype)
    bs = 16
    pasts = np.array([0, 37, 0, 130], np.int64)
    lens = np.array([70, 9, 1, 200], np.int64)
    totals = pasts + lens
    pages = (totals + bs - 1) // bs
    perm = rng.permutation(int(pages.sum()) + 2).astype(np.int32)
    width = int(pages.max())
    table = np.full((4, width), -1, np.int32)
    cur = 0
    for s in range(4):
        table[s, :pages[s]] = perm[cur:cur + pages[s]]
        cur += pages[s]
    layers = 3
    rows_total = (int(pages.sum()) + 2) * bs
    pool = rnd(rng.standard_normal((layers, 2, rows_total, kv_heads, head_dim)).astype(np.float32))
    T = int(lens.sum())
    q, k, v = rnd(rng.standard_normal((3, T, heads, head_dim)).astype(np.float32))
    k, v = k[:, :kv_heads], v[:, :kv_heads]
    positions = np.concatenate([np.arange(p, p + n) for p, n in zip(pasts, lens)]).astype(np.int32)
    seq_of = np.repeat(np.arange(4), lens)
    wrows = np.concatenate([write_rows(table[s], np.arange(p, p + n), bs) for s, (p, n) in enumerate(zip(pasts, lens))])
    style = 1 if dtype == "bf16" else 2
    cos, sin = rope_tables(head_dim, 10000.0, int(totals.max()), style, dtype)
    layer = 1
    # Oracle: rotate, write, attend.
    q_rot = apply_rope(q, cos[positions], sin[positions], style, dtype)
    k_rot = apply_rope(k, cos[positions], sin[positions], style, dtype)
    want_pool = pool.copy()
    want_pool[layer, 0, wrows] = k_rot
    want_pool[layer, 1, wrows] = v
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    want = prefill_attention(q_rot, want_pool, layer, table, np.arange(4), cu, pasts, bs, head_dim ** -0.5, dtype)
    # HIP.
    pt = dev(pool, DT[dtype]).contiguous()
    view = ops.KVPoolView(pt, bs)
    qo = torch.empty((T, heads, head_dim), dtype=DT[dtype], device="cuda")
    ops.rope_kv_write_raw(dev(q, DT[dtype]), dev(k, DT[dtype]), dev(v, DT[dtype]), qo, view, layer, dev(wrows),
                          dev(positions), dev(cos), dev(sin), style, None, None)
    np.testing.assert_array_equal(host(qo), q_rot)
    np.testing.assert_array_equal(host(pt), want_pool)
    # The same write from column slices of one fused [T, (H + 2 Hkv) * D] QKV buffer (the
    # models' layout) reads the tokens in place and must give the same bits.
    fused = torch.cat([dev(q, DT[dtype]).reshape(T, -1), dev(k, DT[dtype]).reshape(T, -1),
                       dev(v, DT[dtype]).reshape(T, -1)], dim=1)
    qw, kw = heads * head_dim, kv_heads * head_dim
    pt2 = dev(pool, DT[dtype]).contiguous()
    qo2 = torch.empty_like(qo)
    ops.rope_kv_write_raw(fused[:, :qw].view(T, heads, head_dim), fused[:, qw:qw + kw].view(T, kv_heads, head_dim),
                          fused[:, qw + kw:].view(T, kv_heads, head_dim), qo2, ops.KVPoolView(pt2, bs), layer,
                          dev(wrows), dev(positions), dev(cos), dev(sin), style, None, None)
    torch.cuda.synchronize()
    assert torch.equal(qo2, qo) and torch.equal(pt2, pt)
    tile_seq, tile_q0 = ops.prefill_tiles(lens, pasts)
    out = torch.empty_like(qo)
    ops.prefill_attention_raw(qo, view, layer, dev(table), dev(np.arange(4, dtype=np.int32)), dev(cu),
                              dev(pasts.astype(np.int32)), dev(tile_seq), dev(tile_q0), out, head_dim ** -0.5)
    got = host(out)
    err = np.abs(got - want)
    max_tol, mean_tol = (2e-2, 2e-3) if dtype == "bf16" else (2e-5, 2e-6)
    assert err.max() <= max_tol, err.max()
    assert err.mean() <= mean_tol, err.mean()
    del seq_of


@pytest.mark.parametrize("dtype,head_dim,heads,kv_heads,q_gain", [("bf16", 128, 4, 4, 1.0), ("bf16", 128, 4, 2, 6.0),
                                                                  ("bf16", 64, 4, 1, 6.0), ("f32", 64, 2, 2, 6.0)])
def test_prefill_attention_long_prefixes(dtype: str, head_dim: int, heads: int, kv_heads: int, q_gain: float) -> None:
    """Prefixes of up to 17k cached positions (past the 1024 block ids a workgroup keeps
    in LDS), chunks that are not whole 128-query tiles, a one-token chunk, and with
    q_gain 6 scores spread wide enough that the running max moves by more than 2^8
    (exp2 units) many times along a row."""

    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(head_dim + kv_heads)
    rnd = rounder(dtype)
    bs = 16
    pasts = np.array([700, 0, 17000, 3000, 255], np.int64)
    lens = np.array([300, 129, 128, 1, 257], np.int64)
    totals = pasts + lens
    pages = (totals + bs - 1) // bs
    perm = rng.permutation(int(pages.sum()) + 3).astype(np.int32)
    table = np.full((lens.size, int(pages.max())), -1, np.int32)
    cur = 0
    for s, n in enumerate(pages):
        table[s, :n] = perm[cur:cur + n]
        cur += n
    rows_total = (int(pages.sum()) + 3) * bs
    pool = rnd(rng.standard_normal((1, 2, rows_total, kv_heads, head_dim)).astype(np.float32))
    q = rnd((q_gain * rng.standard_normal((int(lens.sum()), heads, head_dim))).astype(np.float32))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    scale = head_dim ** -0.5
    want = prefill_attention(q, pool, 0, table, np.arange(lens.size), cu, pasts, bs, scale, dtype)
    view = ops.KVPoolView(dev(pool, DT[dtype]).contiguous(), bs)
    qt = dev(q, DT[dtype])
    tile_seq, tile_q0 = ops.prefill_tiles(lens, pasts)
    out = torch.empty_like(qt)
    ops.prefill_attention_raw(qt, view, 0, dev(table), dev(np.arange(lens.size, dtype=np.int32)), dev(cu),
                              dev(pasts.astype(np.int32)), dev(tile_seq), dev(tile_q0), out, scale)
    # With q_gain 6 an output is close to one value row, up to |v| ~ 4.5, where storing it in
    # bf16 alone moves it by up to half a bf16 step (2^-6 at 4.5). The bound is absolute: 2e-2
    # (2e-5 in fp32) plus that half step of the stored output's own rounding.
    max_tol, mean_tol = (2e-2, 2e-3) if dtype == "bf16" else (2e-5, 2e-6)
    mant = 7 if dtype == "bf16" else 23
    half_step = np.ldexp(0.5, np.frexp(np.maximum(np.abs(want), 1e-30))[1] - 1 - mant)
    bound = max_tol + half_step
    err = np.abs(host(out) - want)
    assert (err <= bound).all(), (err - bound).max()
    assert err.mean() <= mean_tol, err.mean()
    if dtype != "bf16":
        return
    # The same tiles with their key ranges split over workgroups (8 blocks of 32 keys at most,
    # so the 17k-key prefix takes dozens of parts) and merged: the oracle's tolerance again.
    work = ops.prefill_split_work(lens, pasts, num_heads=heads, max_blocks=8)
    assert work.num_slots > 0 and len(work.merges) > 0
    partials = torch.empty(ops.prefill_partial_bytes(work.num_slots, heads, head_dim) // 4, dtype=torch.float32,
                           device="cuda")
    out_split = torch.full_like(qt, float("nan"))
    ops.prefill_attention_split_raw(qt, view, 0, dev(table), dev(np.arange(lens.size, dtype=np.int32)), dev(cu),
                                    dev(pasts.astype(np.int32)), dev(work.items), dev(work.merges), work.num_slots,
                                    partials, out_split, scale)
    err = np.abs(host(out_split) - want)
    assert (err <= bound).all(), (err - bound).max()
    assert err.mean() <= mean_tol, err.mean()


@pytest.mark.parametrize("rows,live", [(1, 1), (8, 5), (256, 256), (512, 300), (1500, 1400)])
def test_route_compact_lists_exits_then_stays_in_launch_order(rows: int, live: int) -> None:
    """cdb_route_compact against its restatement: [n_exit, n_stay, exiting rows, staying rows],
    each list in launch order, padding rows (negative bank slot) in neither; bit-exact."""

    from continuous_depth_batching_amd import ops

    rng = np.random.default_rng(rows)
    flags = (rng.random(rows) < 0.35).astype(np.uint8)
    slots = np.full(rows, -1, np.int64)
    slots[:live] = rng.permutation(4 * rows)[:live]
    lists = torch.full((2 + rows,), -7, dtype=torch.int32, device="cuda")
    torch.ops.cdb.route_compact(dev(flags), dev(slots), lists)
    got = lists.cpu().numpy()
    exits = [r for r in range(rows) if slots[r] >= 0 and flags[r]]
    stays = [r for r in range(rows) if slots[r] >= 0 and not flags[r]]
    want = np.array([len(exits), len(stays)] + exits + stays, np.int32)
    np.testing.assert_array_equal(got[:2 + live], want)
    assert np.all(got[2 + live:] == -7)  # nothing written past the live rows' lists
