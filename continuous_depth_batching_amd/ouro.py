"""Ouro looped LM: random-init module and its CDB adapter on the HIP kernels.

``OuroForCausalLM`` reproduces the reference model's structure and parameter
names (ouro/modeling_ouro.py:156-603, 755-775) so that a state dict of the
reference model loads unchanged: a fully looped decoder whose 4-norm
("sandwich") layers run ``total_ut_steps`` times, split-half RoPE, MHA,
SwiGLU MLP, a final norm after every loop step, and Linear(E, 1) exit gates.

``OuroCDBAdapter`` (cdb/adapters/ouro.py:116-358) runs the CDB stages:
  * prelude = embedding lookup written straight into hidden-bank rows;
  * recurrent step = one pass through the layer stack: fused RMSNorm
    sandwiches, one fused QKV GEMM, the mixed-depth paged decode attention
    with fused RoPE + KV append, O-projection, fused gate/up GEMM + SiLU, down
    GEMM, the final norm, the bank scatter and the exit gate -- all on the
    stream, capturable as one HIP graph per bucket;
  * coda = bank gather, then the LM head with its greedy argmax fused
    (cdb_linear_argmax: the logits never reach memory);
  * prefill = the same stack over prompt tokens with the MFMA varlen attention.
Dense projections of decode batches run on the weight-streaming ``cdb::linear``
kernels (the gated form writes silu(gate) * up directly); the O and down
projections write split-K fp32 partials that the residual norm after them
adds and rounds (``cdb::linear_residual_rmsnorm``); larger batches (prefill)
use torch matmuls (hipBLASLt); the LM head's packed copy serves coda batches
of up to 32 rows.
Everything else is ``torch.ops.cdb.*`` / the C ABI.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

import torch
from torch import nn

from . import ops
from .exit_policy import DecisionHorizon, ExitDecisionRule, ExitPolicySpec
from .kv_cache_policy import DEPTH_INDEXED, LoopedKvLayout
from .model_adapter import CDBModelAdapter, PrefillLaunch, RecurrentLaunch, StageLaunch

EXIT_GATE_TYPES = ("early_exit", "lookahead", "preloop")


@dataclass
class OuroConfig:
    """The Ouro config fields the model and engine read (ouro/configuration_ouro.py:152-177)."""

    vocab_size: int = 49152
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    num_key_value_heads: int = 16
    head_dim: int | None = None
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    max_position_embeddings: int = 65536
    total_ut_steps: int = 4
    initializer_range: float = 0.02
    exit_gate_type: str = "early_exit"
    hidden_act: str = "silu"
    sliding_window: int | None = None
    model_type: str = "ouro"
    _attn_implementation: str = "paged|flash_attention_3"
    layer_types: list[str] = field(default_factory=list)

    def __post_init__(self) -> None:
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads
        if not self.layer_types:
            self.layer_types = ["full_attention"] * self.num_hidden_layers

    @property
    def rope_parameters(self) -> dict[str, Any]:
        return {"rope_type": "default", "rope_theta": self.rope_theta}


class OuroRMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps


class OuroAttention(nn.Module):
    def __init__(self, config: OuroConfig, layer_idx: int) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.head_dim = config.head_dim
        self.scaling = self.head_dim ** -0.5
        e, h, hkv = config.hidden_size, config.num_attention_heads, config.num_key_value_heads
        self.q_proj = nn.Linear(e, h * self.head_dim, bias=False)
        self.k_proj = nn.Linear(e, hkv * self.head_dim, bias=False)
        self.v_proj = nn.Linear(e, hkv * self.head_dim, bias=False)
        self.o_proj = nn.Linear(h * self.head_dim, e, bias=False)


class OuroMLP(nn.Module):
    def __init__(self, config: OuroConfig) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)


class OuroDecoderLayer(nn.Module):
    def __init__(self, config: OuroConfig, layer_idx: int) -> None:
        super().__init__()
        self.self_attn = OuroAttention(config, layer_idx)
        self.mlp = OuroMLP(config)
        self.input_layernorm = OuroRMSNorm(config.hidden_size, config.rms_norm_eps)
        self.input_layernorm_2 = OuroRMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = OuroRMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm_2 = OuroRMSNorm(config.hidden_size, config.rms_norm_eps)


class OuroModel(nn.Module):
    def __init__(self, config: OuroConfig) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(OuroDecoderLayer(config, i) for i in range(config.num_hidden_layers))
        self.norm = OuroRMSNorm(config.hidden_size, config.rms_norm_eps)
        self.total_ut_steps = config.total_ut_steps
        self.early_exit_gate = nn.Linear(config.hidden_size, 1)
        self.lookahead_exit_gate = nn.Linear(config.hidden_size, 1)
        self.preloop_exit_gate = nn.Linear(config.hidden_size, config.total_ut_steps)


class OuroForCausalLM(nn.Module):
    def __init__(self, config: OuroConfig) -> None:
        super().__init__()
        self.config = config
        self.model = OuroModel(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)

    def get_decoder(self) -> OuroModel:
        return self.model


def ouro_1p4b_config(num_hidden_layers: int = 24) -> OuroConfig:
    """The Ouro-1.4B shape (48 layers: the Ouro-2.6B shape): hidden 2048, 16 heads x 128, MLP 5632,
    vocab 49152, 4 loop steps."""

    return OuroConfig(vocab_size=49152, hidden_size=2048, intermediate_size=5632,
                      num_hidden_layers=num_hidden_layers, num_attention_heads=16, num_key_value_heads=16,
                      head_dim=128, total_ut_steps=4, max_position_embeddings=16384)


def init_ouro_weights(model: OuroForCausalLM, *, seed: int, std: float | None = None) -> OuroForCausalLM:
    """Random init: Linear/Embedding weights N(0, std), biases 0, RMSNorm weights 1, drawn from one
    seeded generator on the model's device in a fixed parameter order."""

    std = model.config.initializer_range if std is None else std
    device = next(model.parameters()).device
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("layernorm.weight") or name.endswith("layernorm_2.weight") or name.endswith("norm.weight"):
                p.fill_(1.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                tmp = torch.empty(p.shape, dtype=torch.float32, device=device)
                tmp.normal_(0.0, std, generator=gen)
                p.copy_(tmp)
    return model


def build_ouro(config: OuroConfig, *, seed: int, dtype: torch.dtype, device: torch.device | str) -> OuroForCausalLM:
    with torch.device(device):
        model = OuroForCausalLM(config)
    init_ouro_weights(model, seed=seed)
    return model.to(dtype).eval()


def rope_tables(head_dim: int, theta: float, max_positions: int, dtype: torch.dtype,
                device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [max_positions, D/2] as the rotary module computes them (ouro/modeling_ouro.py:544-573):
    fp32 angles inv_freq * position, cast to the model dtype; stored as fp32 for the kernels."""

    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(device=device,
                                                                                  dtype=torch.float) / head_dim))
    pos = torch.arange(max_positions, device=device, dtype=torch.float32)
    freqs = (inv_freq[:, None] @ pos[None, :]).transpose(0, 1)
    return freqs.cos().to(dtype).float().contiguous(), freqs.sin().to(dtype).float().contiguous()


class OuroCDBAdapter(CDBModelAdapter):
    """Stage kernels for Ouro; weights are packed once (fused QKV and gate/up)."""

    coda_writes_successor_prelude = True  # the prelude is the embedding lookup the coda can fuse

    def __init__(self, model: nn.Module, *, max_positions: int | None = None) -> None:
        self.model = model
        self.decoder = model.get_decoder() if hasattr(model, "get_decoder") else model.model
        cfg = self.decoder.config
        self.config = cfg
        gate_type = "early_exit" if getattr(cfg, "exit_gate_type", "early_exit") == "same_step" else \
            getattr(cfg, "exit_gate_type", "early_exit")
        if gate_type not in EXIT_GATE_TYPES:
            raise NotImplementedError(f"unsupported exit_gate_type {gate_type!r}")
        if gate_type == "preloop":
            raise NotImplementedError("the preloop exit gate is not served by this engine")
        self._gate_type = gate_type
        gate = self.decoder.lookahead_exit_gate if gate_type == "lookahead" else self.decoder.early_exit_gate
        p = next(model.parameters())
        self._dtype, self._device = p.dtype, p.device
        e = cfg.hidden_size
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = cfg.head_dim or e // self.num_heads
        self.eps = float(cfg.rms_norm_eps)
        self.q_width = self.num_heads * self.head_dim
        self.kv_width = self.num_kv_heads * self.head_dim
        with torch.no_grad():
            self.layers = []
            for layer in self.decoder.layers[: cfg.num_hidden_layers]:
                at, mlp = layer.self_attn, layer.mlp
                self.layers.append(dict(
                    wqkv=torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight], 0).contiguous(),
                    wo=at.o_proj.weight.contiguous(),
                    wgu=torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight], 0).contiguous(),
                    wd=mlp.down_proj.weight.contiguous(),
                    n_in=layer.input_layernorm.weight.contiguous(),
                    n_in2=layer.input_layernorm_2.weight.contiguous(),
                    n_post=layer.post_attention_layernorm.weight.contiguous(),
                    n_post2=layer.post_attention_layernorm_2.weight.contiguous(),
                ))
            # Operand-ordered copies for the decode-batch projection kernel.
            for w in self.layers:
                for name in ("wqkv", "wo", "wgu", "wd"):
                    w["p" + name[1:]] = ops.maybe_pack_linear_weight(w[name])
            self.final_norm = self.decoder.norm.weight.contiguous()
            self.gate_w = gate.weight.reshape(-1).contiguous()
            self.gate_b = gate.bias.reshape(-1).contiguous() if gate.bias is not None else None
            self.embed = self.decoder.embed_tokens.weight
            self.lm_head_w = model.lm_head.weight
            self.lm_head_p = ops.maybe_pack_linear_weight(self.lm_head_w)
        positions = max_positions or int(getattr(cfg, "max_position_embeddings", 65536))
        self.rope_cos, self.rope_sin = rope_tables(self.head_dim, float(cfg.rope_theta), positions, self._dtype,
                                                   self._device)
        self.scale = self.head_dim ** -0.5
        self.kv_policy = DEPTH_INDEXED
        self.kv_slots_per_layer: int | None = None
        self.total_ut_steps = int(cfg.total_ut_steps)

    @staticmethod
    def supports(model: nn.Module) -> bool:
        decoder = model.get_decoder() if hasattr(model, "get_decoder") else getattr(model, "model", model)
        kinds = {getattr(getattr(model, "config", None), "model_type", None),
                 getattr(getattr(decoder, "config", None), "model_type", None)}
        return "ouro" in kinds and all(hasattr(decoder, n) for n in ("embed_tokens", "layers", "norm")) \
            and hasattr(model, "lm_head")

    # -- configuration -------------------------------------------------------------------------------------------
    @property
    def hidden_width(self) -> int:
        return self.config.hidden_size

    @property
    def dtype(self) -> torch.dtype:
        return self._dtype

    @property
    def device(self) -> torch.device:
        return self._device

    def configure_recurrent_steps(self, max_recurrent_steps: int) -> None:
        self.total_ut_steps = max_recurrent_steps
        self.config.total_ut_steps = max_recurrent_steps

    def configure_kv_policy(self, kv_policy: str, kv_slots_per_layer: int | None) -> None:
        self.kv_policy = kv_policy
        self.kv_slots_per_layer = kv_slots_per_layer

    def kv_cache_layout(self) -> LoopedKvLayout:
        return LoopedKvLayout.build(num_prelude_layers=0, num_core_layers=self.config.num_hidden_layers,
                                    num_coda_layers=0, total_recurrent_steps=self.total_ut_steps,
                                    policy=self.kv_policy, requested_slots=self.kv_slots_per_layer)

    def kv_geometry(self) -> tuple[int, int]:
        return self.num_kv_heads, self.head_dim

    def exit_policy_spec(self) -> ExitPolicySpec:
        horizon = DecisionHorizon.OFFSET_ONE if self._gate_type == "lookahead" else DecisionHorizon.SAME_STEP
        return ExitPolicySpec(ExitDecisionRule.CUMULATIVE_HAZARD, horizon)

    def gate_params(self) -> tuple[int, torch.Tensor, torch.Tensor | None]:
        return ops.GATE_HAZARD, self.gate_w, self.gate_b

    # -- stages --------------------------------------------------------------------------------------------------
    def prelude(self, launch: StageLaunch) -> None:
        ops.copy_rows_raw(self.embed, launch.tokens, launch.bank, launch.slots, launch.n)

    def _layer_stack(self, x: torch.Tensor, residual: torch.Tensor, attend) -> torch.Tensor:
        """Run every layer; x = input_layernorm(residual) on entry. Returns the final-normed hidden."""

        num_layers = len(self.layers)
        rows = x.shape[0]
        for li, w in enumerate(self.layers):
            qkv = ops.linear_auto(x, w["wqkv"], w["pqkv"], False)
            attn = attend(li, qkv)
            residual, x = ops.linear_residual_rmsnorm_auto(attn.view(rows, self.q_width), w["wo"], w["po"], residual,
                                                           w["n_in2"], w["n_post"], self.eps, self.eps,
                                                           ops.NORM_OURO_SANDWICH)
            act = ops.linear_auto(x, w["wgu"], w["pgu"], True)
            nxt = self.layers[li + 1]["n_in"] if li + 1 < num_layers else self.final_norm
            residual, x = ops.linear_residual_rmsnorm_auto(act, w["wd"], w["pd"], residual, w["n_post2"], nxt,
                                                           self.eps, self.eps, ops.NORM_OURO_SANDWICH)
        return x

    def recurrent_step(self, launch: RecurrentLaunch) -> None:
        rows = launch.rows
        cache = launch.cache
        residual = torch.ops.cdb.gather_rows(launch.bank, launch.bank_slots)
        x = torch.ops.cdb.rmsnorm(residual, self.layers[0]["n_in"], self.eps)
        q_w, kv_w = self.q_width, self.kv_width
        hd = self.head_dim

        def attend(li: int, qkv: torch.Tensor) -> torch.Tensor:
            q = qkv[:, :q_w].view(rows, self.num_heads, hd)
            k = qkv[:, q_w:q_w + kv_w].view(rows, self.num_kv_heads, hd)
            v = qkv[:, q_w + kv_w:].view(rows, self.num_kv_heads, hd)
            # Every layer serves the same rows: the first one plans their chunks.
            return torch.ops.cdb.paged_decode_attention(
                q, k, v, cache.pool, launch.slot_offset, li, cache.device_table, launch.table_rows,
                launch.positions, self.rope_cos, self.rope_sin, 1, None, None, launch.workspace,
                cache.block_size, launch.split_pages, self.scale,
                ops.DECODE_PLAN_AND_ATTEND if li == 0 else ops.DECODE_ATTEND)

        hidden = self._layer_stack(x, residual, attend)
        torch.ops.cdb.scatter_rows_(launch.bank, launch.bank_slots, hidden)
        g = launch.gate
        if g.enabled:
            kind, w, b = self.gate_params()
            torch.ops.cdb.exit_gate(hidden, None, w, b, g.signal, g.state.cdf, g.state.survival, g.state.pending,
                                    launch.bank_slots, g.steps, g.synthetic, g.flags, rows, kind, g.rule, False,
                                    g.round_hazard, g.min_steps, g.max_steps, g.threshold)

    def prefill(self, launch: PrefillLaunch) -> torch.Tensor:
        cache = launch.cache
        tokens = launch.tokens.numel()
        hidden = torch.ops.cdb.gather_rows(self.embed, launch.tokens)
        layout = self.kv_cache_layout()
        q_w, kv_w, hd = self.q_width, self.kv_width, self.head_dim
        for ut in range(self.total_ut_steps):
            residual = hidden
            x = torch.ops.cdb.rmsnorm(residual, self.layers[0]["n_in"], self.eps)

            def attend(li: int, qkv: torch.Tensor, ut: int = ut) -> torch.Tensor:
                layer = layout.core_layer_index(li, ut)
                # Strided column slices of the fused QKV output: no split copies.
                q = qkv[:, :q_w].view(tokens, self.num_heads, hd)
                k = qkv[:, q_w:q_w + kv_w].view(tokens, self.num_kv_heads, hd)
                v = qkv[:, q_w + kv_w:].view(tokens, self.num_kv_heads, hd)
                q_rot = torch.ops.cdb.rope_kv_write(q, k, v, cache.pool, layer, cache.block_size, launch.write_rows,
                                                    launch.positions, self.rope_cos, self.rope_sin, 1, None, None)
                return ops.prefill_attention_launch(q_rot, cache.pool, layer, cache.block_size, cache.device_table,
                                                    launch, self.scale)

            hidden = self._layer_stack(x, residual, attend)
        last = torch.ops.cdb.gather_rows(hidden, launch.last_index)
        return self.coda_from_hidden(last)

    def coda_weights(self) -> ops.CodaWeights | None:
        # The coda is the LM head + argmax of the bank rows (the final norm is applied at
        # the end of every loop step), so the direct call computes exactly coda().
        if self.lm_head_p is None or self._dtype is not torch.bfloat16 or self.lm_head_w.shape[0] % 16:
            return None
        return ops.CodaWeights(packed=self.lm_head_p, vocab=self.lm_head_w.shape[0], width=self.lm_head_w.shape[1],
                               embed=self.embed.contiguous())

    def coda_from_hidden(self, hidden: torch.Tensor) -> torch.Tensor:
        return ops.lm_head_argmax(hidden, self.lm_head_w, self.lm_head_p)

    def coda(self, launch: StageLaunch) -> torch.Tensor:
        # Eager, once per coda tick: direct calls rather than op dispatch. Rows with an
        # eager successor also get its prelude -- the embedding of the greedy token in
        # the successor's bank slot -- from the same launch.
        hidden = ops.gather_rows_raw(launch.bank, launch.slots[:launch.n])
        if launch.successor_slots is None:
            return self.coda_from_hidden(hidden)
        return ops.lm_head_argmax(hidden, self.lm_head_w, self.lm_head_p, embed=self.embed, bank=launch.bank,
                                  bank_slots=launch.successor_slots)


__all__ = ["OuroConfig", "OuroForCausalLM", "OuroCDBAdapter", "build_ouro", "init_ouro_weights", "rope_tables",
           "math"]
