"""The one-call greedy coda (cdb_coda_greedy) against the same coda as separate calls.

The direct call uploads the coda rows' bank slots (and their successors' slots), gathers the
rows, runs the LM head with the fused argmax (writing each successor's embedding row) and
resets the successors' gate state. Each part is an existing entry point, so tokens, bank rows
and gate state must equal the multi-call path's bit for bit, including when a turn's buffers
are reused by a smaller coda right after a larger one.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

VOCAB, WIDTH, BANK_ROWS = 4096, 2048, 256


@pytest.fixture(scope="module")
def setup():
    from continuous_depth_batching_amd import ops

    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    bank = torch.randn((BANK_ROWS, WIDTH), generator=g, device="cuda").bfloat16()
    w = (torch.randn((VOCAB, WIDTH), generator=g, device="cuda") * 0.02).bfloat16()
    embed = torch.randn((VOCAB, WIDTH), generator=g, device="cuda").bfloat16()
    packed = ops.pack_linear_weight(w)
    weights = ops.CodaWeights(packed=packed, vocab=VOCAB, width=WIDTH, embed=embed)
    return ops, bank, w, packed, embed, weights


def _gate_state(ops, capacity: int, seed: int):
    state = ops.GateState.allocate(capacity, torch.device("cuda"))
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    state.cdf.copy_(torch.rand(capacity, generator=g, device="cuda", dtype=torch.float64))
    state.survival.copy_(torch.rand(capacity, generator=g, device="cuda", dtype=torch.float64))
    state.pending.copy_(torch.rand(capacity, generator=g, device="cuda"))
    return state


@pytest.mark.parametrize("fused", [True, False])
def test_direct_coda_equals_the_separate_calls(setup, fused: bool) -> None:
    ops, bank0, w, packed, embed, weights = setup
    host_upload = torch.empty(3 * 256, dtype=torch.int64, pin_memory=True)
    dev_upload = torch.empty(3 * 256, dtype=torch.int64, device="cuda")
    host_tokens = torch.empty(256, dtype=torch.int64, pin_memory=True)
    bank_direct = bank0.clone()
    state_direct = _gate_state(ops, BANK_ROWS, 5)
    scratch = ops.CodaScratch(weights, bank_direct, state_direct, host_upload, dev_upload, host_tokens)
    bank_ref = bank0.clone()
    state_ref = _gate_state(ops, BANK_ROWS, 5)
    stream = torch.cuda.current_stream().cuda_stream
    # Two codas in a row on the same turn buffers, the second smaller.
    for call, rows in enumerate((32, 7)):
        print(f"[direct coda] fused={fused} call {call} rows {rows}", flush=True)
        slots = torch.randperm(128, device="cuda")[:rows].to(torch.int64)
        succ = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
        with_successor = torch.arange(0, rows, 2, device="cuda") if fused else torch.zeros(0, dtype=torch.long,
                                                                                               device="cuda")
        new_slots = 128 + 40 * call + torch.arange(with_successor.numel(), device="cuda", dtype=torch.int64)
        succ[with_successor] = new_slots
        n_succ = int(with_successor.numel())
        upload = torch.cat([slots, succ, new_slots]) if fused else slots
        host_upload[:upload.numel()].copy_(upload.cpu())
        scratch.launch(rows, n_succ, fused, stream)
        torch.cuda.synchronize()
        got = host_tokens[:rows].clone()
        assert torch.equal(scratch.tokens[:rows].cpu(), got)

        hidden = ops.gather_rows_raw(bank_ref, slots)
        if fused:
            want = ops.lm_head_argmax(hidden, w, packed, embed=embed, bank=bank_ref, bank_slots=succ)
            state_ref.reset(new_slots, n_succ)
        else:
            want = ops.lm_head_argmax(hidden, w, packed)
        torch.cuda.synchronize()
        assert torch.equal(got, want.cpu())
        assert torch.equal(bank_direct, bank_ref)
        for name in ("cdf", "survival", "pending"):  # a reset leaves pending NaN (no signal yet)
            torch.testing.assert_close(getattr(state_direct, name), getattr(state_ref, name), rtol=0, atol=0,
                                       equal_nan=True, msg=name)
        if fused:
            assert torch.equal(bank_direct[new_slots], embed[want[with_successor]])
            assert bool((state_direct.cdf[new_slots] == 0).all()) and bool((state_direct.survival[new_slots] == 1).all())


def test_direct_coda_rejects_rows_beyond_its_buffers(setup) -> None:
    ops, bank0, _w, _packed, _embed, weights = setup
    host_upload = torch.empty(3 * 64, dtype=torch.int64, pin_memory=True)
    dev_upload = torch.empty(3 * 64, dtype=torch.int64, device="cuda")
    host_tokens = torch.empty(64, dtype=torch.int64, pin_memory=True)
    scratch = ops.CodaScratch(weights, bank0.clone(), _gate_state(ops, BANK_ROWS, 1), host_upload, dev_upload,
                              host_tokens)
    with pytest.raises(ValueError):
        scratch.launch(ops.CODA_DIRECT_MAX_ROWS + 1, 0, False, torch.cuda.current_stream().cuda_stream)
    with pytest.raises(ValueError):
        scratch.launch(0, 0, False, torch.cuda.current_stream().cuda_stream)
