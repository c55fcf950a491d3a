"""Huginn looped LM (prelude / recurrent core / coda) and its CDB adapter on the HIP kernels.

``HuginnForCausalLM`` reproduces the reference model's structure and parameter
names (huginn/modeling_huginn.py:223-505, configuration_huginn.py:22-141) so a
reference state dict loads unchanged:
  * token embeddings scaled by sqrt(n_embd);
  * sandwich blocks ``x1 = norm_2(attn(norm_1(x)) + x); out = norm_4(mlp(norm_3(x1)) + x1)``;
  * fused Wqkv, a learned per-head qk_bias added before interleaved-pair RoPE
    (theta 50000, fp32 rotation, one rounding);
  * the core input ``adapter(cat(state, injection))`` at every recurrent step;
  * coda = ``ln_f -> coda blocks -> ln_f``, LM head tied to the embedding.

``HuginnCDBAdapter`` (cdb/adapters/huginn.py:42-189) runs the CDB stages. The
prelude and coda attend over their own KV (``stages_use_attention``):
  * prelude: embedding * sqrt(E), prelude blocks with paged decode attention at
    the token's position; the injection goes to the adapter's injection bank,
    the recurrent state (zero init) to the hidden bank, both at the item's slot;
  * recurrent step: gather state and injection, one adapter GEMM over the
    interleaved [state | injection] rows, core blocks with the mixed-depth paged
    decode attention (the cache layer follows each row's loop slot), the
    latent-difference exit gate against the previous state, bank scatter;
  * coda: ln_f, coda blocks with paged decode attention, ln_f, LM head, argmax;
  * prefill: the full-depth forward over prompt tokens with the MFMA varlen
    attention, writing prelude, every core slot and coda KV.
The reference packs [state | injection] into one 2E-wide bank row; here the
injection lives in its own bank indexed by the same slot, so the hidden bank
holds the state alone and the exit gate reads the previous state contiguously.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
from torch import nn

from . import ops
from .exit_policy import ExitDecisionRule, ExitPolicySpec
from .kv_cache_policy import DEPTH_INDEXED, LoopedKvLayout
from .model_adapter import CDBModelAdapter, PrefillLaunch, RecurrentLaunch, StageLaunch

ROPE_INTERLEAVED = 2


@dataclass
class HuginnConfig:
    """The Huginn config fields the model and engine read (configuration_huginn.py:44-113)."""

    n_embd: int = 5280
    n_heads: int = 55
    n_layers: int = 8
    n_layers_in_prelude: int = 2
    n_layers_in_recurrent_block: int = 4
    n_layers_in_coda: int = 2
    mean_recurrence: int = 32
    total_recurrent_steps: int | None = None
    block_size: int = 4096
    vocab_size: int = 65536
    intermediate_size: int = 17920
    norm_eps: float = 1e-6
    rope_base: float = 50_000.0
    qk_bias: bool = True
    bias: bool = False
    tie_embeddings: bool = True
    state_init: str = "zero"
    # Seed of the generator behind state_init="random" (None: torch's default generator, as the
    # reference draws it).
    state_seed: int | None = None
    bos_token_id: int = 65504
    eos_token_id: int = 65505
    pad_token_id: int = 65509
    model_type: str = "huginn"
    _attn_implementation: str = "paged|flash_attention_3"
    layer_types: list[str] = field(default_factory=list)

    def __post_init__(self) -> None:
        if self.total_recurrent_steps is None:
            self.total_recurrent_steps = self.mean_recurrence
        expected = self.n_layers_in_prelude + self.n_layers_in_recurrent_block + self.n_layers_in_coda
        if expected != self.n_layers:
            raise ValueError(f"n_layers={self.n_layers} must equal prelude + core + coda = {expected}")
        if self.total_recurrent_steps <= 0:
            raise ValueError(f"total_recurrent_steps must be positive, got {self.total_recurrent_steps}")
        if not self.layer_types:
            self.layer_types = ["full_attention"] * self.n_layers

    # Names the shared engine code reads (the reference maps them with attribute_map).
    @property
    def hidden_size(self) -> int:
        return self.n_embd

    @property
    def num_attention_heads(self) -> int:
        return self.n_heads

    @property
    def num_key_value_heads(self) -> int:
        return self.n_heads

    @property
    def num_hidden_layers(self) -> int:
        return self.n_layers

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_heads

    @property
    def padded_vocab_size(self) -> int:
        return self.vocab_size

    @property
    def sliding_window(self) -> None:
        return None

    @property
    def embed_scale(self) -> float:
        return math.sqrt(self.n_embd)

    @property
    def state_init_std(self) -> float:
        return math.sqrt(2 / (5 * self.n_embd))


class HuginnRMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))


class HuginnAttention(nn.Module):
    def __init__(self, config: HuginnConfig) -> None:
        super().__init__()
        e, h, d = config.n_embd, config.n_heads, config.head_dim
        self.Wqkv = nn.Linear(e, e + 2 * config.num_key_value_heads * d, bias=False)
        if config.qk_bias:
            self.qk_bias = nn.Parameter(torch.zeros(2, 1, h, d))
        self.proj = nn.Linear(e, e, bias=False)


class HuginnMLP(nn.Module):
    def __init__(self, config: HuginnConfig) -> None:
        super().__init__()
        self.fc = nn.Linear(config.n_embd, config.intermediate_size * 2, bias=False)
        self.proj = nn.Linear(config.intermediate_size, config.n_embd, bias=False)


class HuginnBlock(nn.Module):
    def __init__(self, config: HuginnConfig) -> None:
        super().__init__()
        self.norm_1 = HuginnRMSNorm(config.n_embd, config.norm_eps)
        self.attn = HuginnAttention(config)
        self.norm_2 = HuginnRMSNorm(config.n_embd, config.norm_eps)
        self.mlp = HuginnMLP(config)
        self.norm_3 = HuginnRMSNorm(config.n_embd, config.norm_eps)
        self.norm_4 = HuginnRMSNorm(config.n_embd, config.norm_eps)


class HuginnForCausalLM(nn.Module):
    def __init__(self, config: HuginnConfig) -> None:
        super().__init__()
        self.config = config
        self.transformer = nn.ModuleDict({
            "wte": nn.Embedding(config.padded_vocab_size, config.n_embd),
            "prelude": nn.ModuleList(HuginnBlock(config) for _ in range(config.n_layers_in_prelude)),
            "adapter": nn.Linear(config.n_embd * 2, config.n_embd, bias=config.bias),
            "core_block": nn.ModuleList(HuginnBlock(config) for _ in range(config.n_layers_in_recurrent_block)),
            "coda": nn.ModuleList(HuginnBlock(config) for _ in range(config.n_layers_in_coda)),
            "ln_f": HuginnRMSNorm(config.n_embd, config.norm_eps),
        })
        self.lm_head = nn.Linear(config.n_embd, config.padded_vocab_size, bias=False)
        if config.tie_embeddings:
            self.lm_head.weight = self.transformer["wte"].weight


def init_huginn_weights(model: HuginnForCausalLM, *, seed: int, std: float = 0.02,
                        qk_bias_std: float = 0.0) -> HuginnForCausalLM:
    """Random init: Linear/Embedding weights N(0, std), biases 0, RMSNorm weights 1, qk_bias
    N(0, qk_bias_std); one seeded generator on the model's device, fixed parameter order."""

    device = next(model.parameters()).device
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm_1.weight") or name.endswith("norm_2.weight") or name.endswith("norm_3.weight") \
                    or name.endswith("norm_4.weight") or name.endswith("ln_f.weight"):
                p.fill_(1.0)
            elif name.endswith(".bias"):
                p.zero_()
            elif name.endswith("qk_bias"):
                tmp = torch.empty(p.shape, dtype=torch.float32, device=device)
                tmp.normal_(0.0, qk_bias_std, generator=gen) if qk_bias_std > 0 else tmp.zero_()
                p.copy_(tmp)
            else:
                tmp = torch.empty(p.shape, dtype=torch.float32, device=device)
                tmp.normal_(0.0, std, generator=gen)
                p.copy_(tmp)
    return model


def build_huginn(config: HuginnConfig, *, seed: int, dtype: torch.dtype, device: torch.device | str,
                 std: float = 0.02, qk_bias_std: float = 0.0) -> HuginnForCausalLM:
    with torch.device(device):
        model = HuginnForCausalLM(config)
    init_huginn_weights(model, seed=seed, std=std, qk_bias_std=qk_bias_std)
    return model.to(dtype).eval()


def huginn_rope_tables(head_dim: int, theta: float, max_positions: int,
                       device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [max_positions, D/2] in fp32, computed like freqs_cis_for_positions
    (huginn/modeling_huginn.py:150-175): fp32 inverse frequencies, fp32 angle
    position * inv_freq, fp32 cos/sin (no rounding to the model dtype)."""

    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    freqs = torch.arange(max_positions, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    return freqs.cos().contiguous(), freqs.sin().contiguous()


class HuginnCDBAdapter(CDBModelAdapter):
    """Stage kernels for Huginn; block weights are packed once."""

    stages_use_attention = True

    def __init__(self, model: nn.Module, *, max_positions: int | None = None) -> None:
        if not self.supports(model):
            raise TypeError(f"HuginnCDBAdapter does not support model type {type(model)!r}")
        cfg = model.config
        if cfg.state_init not in ("zero", "random"):
            raise ValueError(f"state_init must be 'zero' or 'random', got {cfg.state_init!r}")
        self.model = model
        self.config = cfg
        p = next(model.parameters())
        self._dtype, self._device = p.dtype, p.device
        self._state_generator: torch.Generator | None = None
        if cfg.state_init == "random" and cfg.state_seed is not None:
            self._state_generator = torch.Generator(device=self._device)
            self._state_generator.manual_seed(cfg.state_seed)
        self.E = cfg.n_embd
        self.num_heads = cfg.n_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = cfg.head_dim
        self.eps = float(cfg.norm_eps)
        self.q_width = self.num_heads * self.head_dim
        self.kv_width = self.num_kv_heads * self.head_dim
        self.embed_scale = cfg.embed_scale
        tr = model.transformer
        with torch.no_grad():
            self.prelude_blocks = [self._pack_block(b) for b in tr["prelude"]]
            self.core_blocks = [self._pack_block(b) for b in tr["core_block"]]
            self.coda_blocks = [self._pack_block(b) for b in tr["coda"]]
            self.adapter_w = tr["adapter"].weight.contiguous()
            self.adapter_p = ops.maybe_pack_linear_weight(self.adapter_w)
            self.adapter_b = tr["adapter"].bias.contiguous() if tr["adapter"].bias is not None else None
            self.ln_f = tr["ln_f"].weight.contiguous()
            self.embed = tr["wte"].weight
            self.lm_head_w = model.lm_head.weight
            self.lm_head_p = ops.maybe_pack_linear_weight(self.lm_head_w)
        positions = max_positions or int(getattr(cfg, "block_size", 4096))
        self.max_positions = positions
        self.rope_cos, self.rope_sin = huginn_rope_tables(self.head_dim, float(cfg.rope_base), positions,
                                                          self._device)
        self.scale = self.head_dim ** -0.5
        self.kv_policy = DEPTH_INDEXED
        self.kv_slots_per_layer: int | None = None
        self.total_recurrent_steps = int(cfg.total_recurrent_steps)
        self.injection_bank: torch.Tensor | None = None
        self._interleave: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}

    def _pack_block(self, b: HuginnBlock) -> dict[str, torch.Tensor | None]:
        at = b.attn
        qk = getattr(at, "qk_bias", None)
        w = dict(
            wqkv=at.Wqkv.weight.contiguous(), wo=at.proj.weight.contiguous(),
            wgu=b.mlp.fc.weight.contiguous(), wd=b.mlp.proj.weight.contiguous(),
            n1=b.norm_1.weight.contiguous(), n2=b.norm_2.weight.contiguous(),
            n3=b.norm_3.weight.contiguous(), n4=b.norm_4.weight.contiguous(),
            q_bias=None if qk is None else qk[0, 0].contiguous(),
            k_bias=None if qk is None else qk[1, 0, : self.num_kv_heads].contiguous(),
        )
        # Operand-ordered copies for the decode-batch projection kernel.
        for name in ("wqkv", "wo", "wgu", "wd"):
            w["p" + name[1:]] = ops.maybe_pack_linear_weight(w[name])
        return w

    @staticmethod
    def supports(model: nn.Module) -> bool:
        cfg = getattr(model, "config", None)
        return getattr(cfg, "model_type", None) == "huginn" and hasattr(model, "transformer") \
            and hasattr(model, "lm_head")

    # -- configuration -------------------------------------------------------------------------------------------
    @property
    def hidden_width(self) -> int:
        return self.E

    @property
    def dtype(self) -> torch.dtype:
        return self._dtype

    @property
    def device(self) -> torch.device:
        return self._device

    def configure_recurrent_steps(self, max_recurrent_steps: int) -> None:
        self.total_recurrent_steps = int(max_recurrent_steps)
        self.config.total_recurrent_steps = int(max_recurrent_steps)

    def configure_kv_policy(self, kv_policy: str, kv_slots_per_layer: int | None) -> None:
        self.kv_policy = kv_policy
        self.kv_slots_per_layer = kv_slots_per_layer

    def kv_cache_layout(self) -> LoopedKvLayout:
        c = self.config
        return LoopedKvLayout.build(num_prelude_layers=c.n_layers_in_prelude,
                                    num_core_layers=c.n_layers_in_recurrent_block,
                                    num_coda_layers=c.n_layers_in_coda,
                                    total_recurrent_steps=self.total_recurrent_steps, policy=self.kv_policy,
                                    requested_slots=self.kv_slots_per_layer)

    def kv_geometry(self) -> tuple[int, int]:
        return self.num_kv_heads, self.head_dim

    def exit_policy_spec(self) -> ExitPolicySpec:
        return ExitPolicySpec(ExitDecisionRule.DIRECT_THRESHOLD)

    # -- shared pieces -------------------------------------------------------------------------------------------
    def _norm(self, x: torch.Tensor, w_a: torch.Tensor, w_b: torch.Tensor | None = None,
              residual: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(h, y): h = norm_a(R(residual + x)) (norm_a(x) without residual), y = norm_b(h)."""

        h = torch.empty_like(x)
        y = torch.empty_like(x) if w_b is not None else None
        mode = ops.NORM_HUGINN_SANDWICH if residual is not None else ops.NORM_PLAIN
        ops.rmsnorm_fused_raw(x, residual, w_a, w_b, h, y, mode, self.eps, self.eps)
        return h, y

    def _blocks(self, blocks: list[dict], x: torch.Tensor, n1: torch.Tensor, attend,
                final_norm: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor | None]:
        """Run sandwich blocks on residual x with n1 = norm_1(x); returns (out, final_norm(out))."""

        rows = x.shape[0]
        y_last = None
        for i, w in enumerate(blocks):
            qkv = ops.linear_auto(n1, w["wqkv"], w["pqkv"], False)
            a = attend(i, w, qkv)
            # O and down feed the sandwich norms; shapes with a split-K form hand the norm fp32
            # partials instead of a stored projection.
            x1, y = ops.linear_residual_rmsnorm_auto(a.view(rows, self.q_width), w["wo"], w["po"], x, w["n2"],
                                                     w["n3"], self.eps, self.eps, ops.NORM_HUGINN_SANDWICH)
            act = ops.linear_auto(y, w["wgu"], w["pgu"], True)
            nxt = blocks[i + 1]["n1"] if i + 1 < len(blocks) else final_norm
            x, n1 = ops.linear_residual_rmsnorm_auto(act, w["wd"], w["pd"], x1, w["n4"], nxt, self.eps, self.eps,
                                                     ops.NORM_HUGINN_SANDWICH)
            y_last = n1
        return x, y_last

    def _split_qkv(self, qkv: torch.Tensor, contiguous: bool = False):
        rows = qkv.shape[0]
        q_w, kv_w, hd = self.q_width, self.kv_width, self.head_dim
        q, k, v = qkv[:, :q_w], qkv[:, q_w:q_w + kv_w], qkv[:, q_w + kv_w:]
        if contiguous:
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        return (q.view(rows, self.num_heads, hd), k.view(rows, self.num_kv_heads, hd),
                v.view(rows, self.num_kv_heads, hd))

    def _decode_attend(self, launch_like, layer_of):
        """Paged decode attention at the rows' positions; ``layer_of(i)`` gives (per-row offsets, base)."""

        cache = launch_like.cache
        planned = [False]  # every layer of this launch serves the same rows: the first one plans their chunks

        def attend(i: int, w: dict, qkv: torch.Tensor) -> torch.Tensor:
            q, k, v = self._split_qkv(qkv)
            per_row, base = layer_of(i)
            stages = ops.DECODE_ATTEND if planned[0] else ops.DECODE_PLAN_AND_ATTEND
            planned[0] = True
            return torch.ops.cdb.paged_decode_attention(
                q, k, v, cache.pool, per_row, base, cache.device_table, launch_like.table_rows,
                launch_like.positions, self.rope_cos, self.rope_sin, ROPE_INTERLEAVED, w["q_bias"], w["k_bias"],
                launch_like.workspace, cache.block_size, launch_like.split_pages, self.scale, stages)

        return attend

    def _prefill_attend(self, launch: PrefillLaunch, layer_of):
        cache = launch.cache
        tokens = launch.tokens.numel()

        def attend(i: int, w: dict, qkv: torch.Tensor) -> torch.Tensor:
            layer = layer_of(i)
            q, k, v = self._split_qkv(qkv)  # strided column slices: the kernel reads them in place
            q_rot = torch.ops.cdb.rope_kv_write(q, k, v, cache.pool, layer, cache.block_size, launch.write_rows,
                                                launch.positions, self.rope_cos, self.rope_sin, ROPE_INTERLEAVED,
                                                w["q_bias"], w["k_bias"])
            out = ops.prefill_attention_launch(q_rot, cache.pool, layer, cache.block_size, cache.device_table, launch,
                                               self.scale)
            return out.view(tokens, self.num_heads, self.head_dim)

        return attend

    def _embed(self, tokens: torch.Tensor) -> torch.Tensor:
        # wte(ids) * sqrt(n_embd) in the model dtype (huginn/modeling_huginn.py:431).
        return torch.ops.cdb.gather_rows(self.embed, tokens).mul_(self.embed_scale)

    def _interleave_index(self, rows: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Row indices 2i and 2i+1 that interleave [state | injection] into a [rows, 2E] buffer."""

        idx = self._interleave.get(rows)
        if idx is None:
            even = torch.arange(0, 2 * rows, 2, dtype=torch.int64, device=self._device)
            idx = (even, even + 1)
            self._interleave[rows] = idx
        return idx

    def _core_input(self, state: torch.Tensor, injection_src: torch.Tensor,
                    injection_index: torch.Tensor | None, rows: int) -> torch.Tensor:
        """adapter(cat(state, injection)) as one GEMM over interleaved rows."""

        even, odd = self._interleave_index(rows)
        cat = torch.empty((rows, 2 * self.E), dtype=self._dtype, device=self._device)
        flat = cat.view(2 * rows, self.E)
        ops.copy_rows_raw(state, None, flat, even, rows)
        ops.copy_rows_raw(injection_src, injection_index, flat, odd, rows)
        x = ops.linear_auto(cat, self.adapter_w, self.adapter_p, False)
        if self.adapter_b is not None:
            x = x + self.adapter_b
        return x

    def _ensure_injection_bank(self, bank: torch.Tensor) -> torch.Tensor:
        if self.injection_bank is None or self.injection_bank.shape[0] != bank.shape[0]:
            self.injection_bank = torch.zeros_like(bank)
        return self.injection_bank

    def _initial_state(self, injection: torch.Tensor) -> torch.Tensor:
        """The recurrent state a token starts from (modeling_huginn.py:418-427): zeros, or a
        normal of std sqrt(2 / (5E)) clamped at 3 std and scaled by sqrt(E)."""

        if self.config.state_init == "zero":
            return torch.zeros_like(injection)
        std = self.config.state_init_std
        state = torch.empty_like(injection)
        state.normal_(mean=0.0, std=std, generator=self._state_generator)
        state.clamp_(min=-3 * std, max=3 * std)
        return state.mul_(self.config.embed_scale)

    # -- stages --------------------------------------------------------------------------------------------------
    def prelude(self, launch: StageLaunch) -> None:
        n = launch.n
        inj_bank = self._ensure_injection_bank(launch.bank)
        x = self._embed(launch.tokens[:n])
        layout = self.kv_cache_layout()
        if self.prelude_blocks:
            n1, _ = self._norm(x, self.prelude_blocks[0]["n1"])
            attend = self._decode_attend(launch, lambda i: (None, layout.prelude_layer_index(i)))
            x, _ = self._blocks(self.prelude_blocks, x, n1, attend, None)
        torch.ops.cdb.scatter_rows_(inj_bank, launch.slots[:n], x)
        if self.config.state_init == "random":
            torch.ops.cdb.scatter_rows_(launch.bank, launch.slots[:n], self._initial_state(x))
            return
        # Zero initial state (configuration_huginn.py:31-37, modeling_huginn.py:414-427): a negative
        # source index makes the row copy write zeros.
        minus = torch.full((n,), -1, dtype=torch.int64, device=self._device)
        ops.copy_rows_raw(launch.bank, minus, launch.bank, launch.slots[:n], n)

    def recurrent_step(self, launch: RecurrentLaunch) -> None:
        rows = launch.rows
        inj_bank = self._ensure_injection_bank(launch.bank)
        prev = torch.ops.cdb.gather_rows(launch.bank, launch.bank_slots)
        x = self._core_input(prev, inj_bank, launch.bank_slots, rows)
        n1, _ = self._norm(x, self.core_blocks[0]["n1"])
        attend = self._decode_attend(launch, lambda i: (launch.slot_offset, i))
        state, _ = self._blocks(self.core_blocks, x, n1, attend, None)
        torch.ops.cdb.scatter_rows_(launch.bank, launch.bank_slots, state)
        g = launch.gate
        if g.enabled:
            torch.ops.cdb.exit_gate(state, prev, None, None, g.signal, g.state.cdf, g.state.survival,
                                    g.state.pending, launch.bank_slots, g.steps, g.synthetic, g.flags, rows,
                                    ops.GATE_LATENT_DIFF, g.rule, False, g.round_hazard, g.min_steps, g.max_steps,
                                    g.threshold)

    def _coda_hidden(self, state: torch.Tensor, attend) -> torch.Tensor:
        """ln_f -> coda blocks -> ln_f (huginn/modeling_huginn.py:456-463)."""

        if not self.coda_blocks:
            _, y = self._norm(state, self.ln_f, self.ln_f)
            return y
        x, n1 = self._norm(state, self.ln_f, self.coda_blocks[0]["n1"])
        _, y = self._blocks(self.coda_blocks, x, n1, attend, self.ln_f)
        return y

    def coda(self, launch: StageLaunch) -> torch.Tensor:
        n = launch.n
        state = ops.gather_rows_raw(launch.bank, launch.slots[:n])
        layout = self.kv_cache_layout()
        attend = self._decode_attend(launch, lambda i: (None, layout.coda_layer_index(i)))
        hidden = self._coda_hidden(state, attend)
        return ops.lm_head_argmax(hidden, self.lm_head_w, self.lm_head_p)

    def prefill(self, launch: PrefillLaunch) -> torch.Tensor:
        tokens = launch.tokens.numel()
        layout = self.kv_cache_layout()
        x = self._embed(launch.tokens)
        if self.prelude_blocks:
            n1, _ = self._norm(x, self.prelude_blocks[0]["n1"])
            x, _ = self._blocks(self.prelude_blocks, x, n1,
                                self._prefill_attend(launch, layout.prelude_layer_index), None)
        injection = x
        state = self._initial_state(injection)
        for step in range(self.total_recurrent_steps):
            h = self._core_input(state, injection, None, tokens)
            n1, _ = self._norm(h, self.core_blocks[0]["n1"])
            attend = self._prefill_attend(launch, lambda i, step=step: layout.core_layer_index(i, step))
            state, _ = self._blocks(self.core_blocks, h, n1, attend, None)
        hidden = self._coda_hidden(state, self._prefill_attend(launch, layout.coda_layer_index))
        last = torch.ops.cdb.gather_rows(hidden, launch.last_index)
        return ops.lm_head_argmax(last, self.lm_head_w, self.lm_head_p)


__all__ = ["HuginnConfig", "HuginnForCausalLM", "HuginnCDBAdapter", "build_huginn", "init_huginn_weights",
           "huginn_rope_tables"]
