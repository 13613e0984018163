"""MOSS-Image DiT harness: the producer and caller of the saved tensors the offload hooks see.

The activation-offload engine is op-agnostic, but what it moves (which tensors, in which
order, with which layouts and dtypes) is fixed by the model. This module restates the
reference model's topology and op sequence so that the hooks receive the same saves as they
do under ``training/model.py``: RMSNorm (:154-172), SiTU-GLU (:27-38), half-rotation RoPE
(:41-56, :94-151), joint attention (:59-91) through SDPA (``performance.py:124-160``; packed
sequences ``:163-225``, one SDPA call per sequence on a HIP device, the boolean-mask fallback
on the CPU), the text adapter (:175-242), the single-stream joint block with
shared 6-way modulation (:245-314), the time conditions (:546-567), the per-sample and packed
forwards with the offload context around the traversal (:439-544), and selective
checkpointing (:672-710, :780-789). LoRA follows ``training/lora.py:21-86`` and the int8
weight-only base follows ``training/quantization.py:23-131`` (eager dequantisation).

It is test and benchmark harness code: random-initialised weights, synthetic inputs.
"""

from __future__ import annotations

import math
from typing import Callable

import torch
from torch import nn
from torch.nn import functional as F
from torch.utils.checkpoint import checkpoint

from .activation_offload import activation_cpu_offload


# ---------------------------------------------------------------------------------------------
# elementwise pieces


def situ(hidden: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """SiTU-GLU: ``4 tanh(g/4) sigmoid(g) * 25 tanh(h/25)`` (reference model.py:27-38)."""

    capped_gate = 4.0 * torch.tanh(gate / 4.0) * torch.sigmoid(gate)
    return capped_gate * (25.0 * torch.tanh(hidden / 25.0))


def rotate_rope(tokens: torch.Tensor, rope: torch.Tensor) -> torch.Tensor:
    """Half-rotation RoPE; ``rope`` holds sines then cosines (reference model.py:41-56)."""

    sin, cos = rope.chunk(2, -1)
    sin = torch.cat((sin, sin), -1).unsqueeze(-2)
    cos = torch.cat((cos, cos), -1).unsqueeze(-2)
    first, second = tokens.chunk(2, -1)
    return tokens * cos + torch.cat((-second, first), -1) * sin


def _attention_core(query, key, value, cu_seqlens, seq_lengths=None):
    # performance.py:139-143 (normalised q/k follow the value dtype) and :163-225 (packed
    # sequences). On a HIP device the packed sequences are attended one by one, which is what
    # the reference's varlen kernel computes (performance.py:195-209, flash_attn_varlen_func):
    # PyTorch-ROCm's SDPA with the block-diagonal boolean mask is not repeatable at the text
    # adapter's 1600 packed tokens (its output and q/k gradients change once freed device
    # memory holds other data), so a step without offloading would not reproduce itself. On the
    # CPU the packed sequences are isolated by the reference's block-diagonal boolean mask
    # (:215-225), its portable fallback.
    query = query.to(value.dtype)
    key = key.to(value.dtype)
    if cu_seqlens is None:
        return F.scaled_dot_product_attention(query, key, value)
    if value.device.type == "cuda":
        # the split sizes on the host: passed beside cu_seqlens (a checkpointed block's
        # recomputation gets them that way, since a cu_seqlens restored by the offload hooks is a
        # new tensor), kept on a cu_seqlens built by _cumulative_lengths, or read back from the
        # device (a synchronisation) for one built elsewhere
        lengths = seq_lengths if seq_lengths is not None else getattr(cu_seqlens, "host_lengths", None)
        if lengths is None:
            lengths = (cu_seqlens[1:] - cu_seqlens[:-1]).tolist()
        parts = zip(query.split(lengths, 2), key.split(lengths, 2), value.split(lengths, 2))
        return torch.cat([F.scaled_dot_product_attention(q, k, v) for q, k, v in parts], 2)
    lengths = cu_seqlens[1:] - cu_seqlens[:-1]
    labels = torch.repeat_interleave(
        torch.arange(lengths.numel(), device=value.device), lengths.to(device=value.device, dtype=torch.long)
    )
    mask = labels[:, None].eq(labels[None, :]).unsqueeze(0).unsqueeze(0)
    return F.scaled_dot_product_attention(query, key, value, attn_mask=mask)


def attention(query, key, value, rope, heads, cu_seqlens=None, seq_lengths=None):
    """Joint attention with RoPE on q and k over ``[batch, seq, dim]`` (reference model.py:59-91).
    ``seq_lengths``: the packed sequences' lengths as host integers, when the caller has them."""

    shape = (*query.shape[:2], heads, query.shape[-1] // heads)
    query = rotate_rope(query.reshape(shape), rope).transpose(1, 2)
    key = rotate_rope(key.reshape(shape), rope).transpose(1, 2)
    value = value.reshape(shape).transpose(1, 2)
    mixed = _attention_core(query, key, value, cu_seqlens, seq_lengths)
    return mixed.transpose(1, 2).flatten(2)


def rope_coordinates(images, text_length: int, device) -> torch.Tensor:
    """``(r, t, h, w)`` per token: image grids (centred), then text (reference model.py:94-133)."""

    parts = []
    for reference_index, height, width in images:
        rows, cols = torch.meshgrid(
            torch.arange(height, device=device), torch.arange(width, device=device), indexing="ij"
        )
        grid = torch.stack(
            (torch.full_like(rows, reference_index), torch.full_like(rows, text_length), rows, cols), -1
        ).flatten(0, 1).float()
        grid[:, 2] -= (height - 1) / 2
        grid[:, 3] -= (width - 1) / 2
        parts.append(grid)
    text = torch.zeros(text_length, 4, device=device, dtype=torch.float32)
    text[:, 1] = torch.arange(text_length, device=device)
    return torch.cat((*parts, text), 0)


def rope_phases(coordinates: torch.Tensor, bands: torch.Tensor) -> torch.Tensor:
    """``[1, seq, 8 * bands]``: four sines then four cosines per band (reference model.py:136-151)."""

    phase = coordinates.unsqueeze(-1) * bands.to(device=coordinates.device, dtype=torch.float32)
    return torch.cat((phase.sin(), phase.cos()), -2).flatten(-2).unsqueeze(0)


# ---------------------------------------------------------------------------------------------
# modules


class RMSNorm(nn.Module):
    """fp32 RMSNorm with a learned scale, result in the input dtype (reference model.py:154-172)."""

    def __init__(self, dim: int) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        inv_rms = torch.rsqrt(tokens.float().square().mean(-1, keepdim=True) + 1e-6)
        return (tokens.float() * inv_rms).to(tokens.dtype) * self.weight


def _linear_dtype(module: nn.Module) -> torch.dtype:
    if hasattr(module, "compute_dtype"):
        return module.compute_dtype
    return module.weight.dtype


class TextBlock(nn.Module):
    """Text adapter block with fused qkv (reference model.py:175-215)."""

    def __init__(self, dim: int, ffn_dim: int, heads: int) -> None:
        super().__init__()
        self.heads = heads
        self.norm1, self.norm2 = RMSNorm(dim), RMSNorm(dim)
        self.q_norm, self.k_norm = RMSNorm(dim // heads), RMSNorm(dim // heads)
        self.qkv = nn.Linear(dim, 3 * dim)
        self.proj = nn.Linear(dim, dim)
        self.ffn_gate, self.ffn_up = nn.Linear(dim, ffn_dim), nn.Linear(dim, ffn_dim)
        self.ffn_down = nn.Linear(ffn_dim, dim)

    def forward(self, tokens, rope, cu_seqlens=None):
        query, key, value = self.qkv(self.norm1(tokens)).chunk(3, -1)
        query = self.q_norm(query.unflatten(-1, (self.heads, -1))).flatten(2)
        key = self.k_norm(key.unflatten(-1, (self.heads, -1))).flatten(2)
        tokens = tokens + self.proj(attention(query, key, value, rope, self.heads, cu_seqlens))
        hidden = self.norm2(tokens)
        return tokens + self.ffn_down(situ(self.ffn_up(hidden), self.ffn_gate(hidden)))


class TextProjection(nn.Module):
    """Text-encoder states to DiT width, then two text blocks (reference model.py:218-242)."""

    def __init__(self, text_dim: int, dim: int, ffn_dim: int, heads: int) -> None:
        super().__init__()
        self.proj = nn.Linear(text_dim, dim)
        self.blocks = nn.ModuleList([TextBlock(dim, ffn_dim, heads) for _ in range(2)])

    def forward(self, tokens, rope, cu_seqlens=None):
        hidden = self.proj(tokens.to(_linear_dtype(self.proj)))
        for block in self.blocks:
            hidden = block(hidden, rope, cu_seqlens)
        return hidden


def _modulation_sample_indices(modulation, tokens, cu_seqlens):
    if modulation.shape[0] == tokens.shape[0]:
        return None
    lengths = (cu_seqlens[1:] - cu_seqlens[:-1]).to(dtype=torch.long)
    return torch.repeat_interleave(
        torch.arange(modulation.shape[0], device=modulation.device), lengths, output_size=tokens.shape[1]
    )


def _condition_for_tokens(condition, sample_indices):
    if sample_indices is None:
        return condition[:, None]
    return condition.index_select(0, sample_indices).unsqueeze(0)


MLP_VARIANTS = ("situ", "gelu")


class Block(nn.Module):
    """Joint image/text block with shared scale-shift-gate modulation (reference model.py:245-314).

    ``mlp="situ"`` is the reference block: a fused up/gate projection into SiTU-GLU (:255, :312).
    ``mlp="gelu"`` is the plain GELU MLP (tanh approximation) that BASELINE config 1 names in
    words: ``ffn_up`` [dim -> ffn], GELU, ``ffn_down``. The reference has no such block; it is a
    second producer of saves for the op-agnostic hooks (one bf16/fp32 ``[T, F]`` pre-activation
    per block instead of SiTU's six intermediates).
    """

    def __init__(self, dim: int, ffn_dim: int, heads: int, mlp: str = "situ") -> None:
        super().__init__()
        if mlp not in MLP_VARIANTS:
            raise ValueError(f"mlp must be one of {MLP_VARIANTS}")
        self.heads, self.mlp = heads, mlp
        self.norm1, self.norm2 = RMSNorm(dim), RMSNorm(dim)
        self.q_norm, self.k_norm = RMSNorm(dim // heads), RMSNorm(dim // heads)
        self.proj = nn.ModuleDict({name: nn.Linear(dim, dim, bias=False) for name in ("q", "k", "v", "o")})
        if mlp == "gelu":
            self.proj["ffn_up"] = nn.Linear(dim, ffn_dim, bias=False)
        else:
            self.proj["ffn_up_gate"] = nn.Linear(dim, 2 * ffn_dim, bias=False)
        self.proj["ffn_down"] = nn.Linear(ffn_dim, dim, bias=False)

    def forward(self, tokens, rope, modulation, cu_seqlens=None, seq_lengths=None):
        shift_attn, scale_attn, gate_attn, shift_ffn, scale_ffn, gate_ffn = modulation.unbind(1)
        index = _modulation_sample_indices(modulation, tokens, cu_seqlens)
        hidden = self.norm1(tokens)
        hidden = hidden * (1 + _condition_for_tokens(scale_attn, index))
        hidden = hidden + _condition_for_tokens(shift_attn, index)
        weight_dtype = _linear_dtype(self.proj["q"])
        hidden = hidden.to(weight_dtype)
        query = self.q_norm(self.proj["q"](hidden).unflatten(-1, (self.heads, -1))).flatten(2)
        key = self.k_norm(self.proj["k"](hidden).unflatten(-1, (self.heads, -1))).flatten(2)
        attended = attention(query, key, self.proj["v"](hidden), rope, self.heads, cu_seqlens, seq_lengths)
        tokens = tokens + self.proj["o"](attended) * _condition_for_tokens(gate_attn, index)
        hidden = self.norm2(tokens)
        hidden = hidden * (1 + _condition_for_tokens(scale_ffn, index))
        hidden = hidden + _condition_for_tokens(shift_ffn, index)
        if self.mlp == "gelu":
            activated = F.gelu(self.proj["ffn_up"](hidden.to(weight_dtype)), approximate="tanh")
        else:
            up, gate = self.proj["ffn_up_gate"](hidden.to(weight_dtype)).chunk(2, -1)
            activated = situ(up, gate)
        return tokens + self.proj["ffn_down"](activated) * _condition_for_tokens(gate_ffn, index)


class RoPE(nn.Module):
    """4D RoPE frequencies ``1 / base^(i / bands)`` in fp32 (reference model.py:317-363)."""

    def __init__(self, head_dim: int, base: float) -> None:
        super().__init__()
        self.num_bands = head_dim // 8
        exponent = torch.arange(self.num_bands, dtype=torch.float32) / self.num_bands
        self.register_buffer("bands", 1 / (base**exponent))

    def forward(self, images, text_length, device):
        return rope_phases(rope_coordinates(images, text_length, device), self.bands)


def checkpointed_layer_indices(depth: int, fraction: float) -> frozenset[int]:
    """Nearest-count, evenly spread blocks to recompute (reference model.py:780-789)."""

    value = float(fraction)
    if not 0.0 <= value <= 1.0 or not math.isfinite(value):
        raise ValueError("checkpoint_fraction must be between 0 and 1.")
    count = min(depth, int(depth * value + 0.5))
    if count == 0:
        return frozenset()
    return frozenset(((2 * i + 1) * depth) // (2 * count) for i in range(count))


def _cumulative_lengths(lengths, device):
    cu = torch.tensor([0, *lengths], device=device, dtype=torch.int64).cumsum(0)
    # the split sizes as host integers, so that the per-sequence attention below need not read
    # them back from the device (a synchronisation in every attention call, which would keep
    # the host in step with the GPU for the whole packed traversal)
    cu.host_lengths = tuple(int(n) for n in lengths)
    return cu


class MOSSImageTransformer(nn.Module):
    """Single-stream DiT (reference model.py:366-710), with a swappable offload context.

    ``offload_context`` is the factory called as ``offload_context(model, enabled, device)``
    around each traversal; it defaults to this package's engine-backed
    :func:`activation_cpu_offload`.
    """

    def __init__(
        self,
        dim: int = 3072,
        ffn_dim: int = 8192,
        num_heads: int = 24,
        num_layers: int = 42,
        text_dim: int = 4096,
        freq_dim: int = 256,
        latent_channels: int = 128,
        rope_base: float = 10000.0,
        gradient_checkpointing: bool = False,
        checkpoint_fraction: float = 1.0,
        activation_offload: bool = False,
        mlp: str = "situ",
    ) -> None:
        super().__init__()
        if dim % num_heads or (dim // num_heads) % 8 or freq_dim % 2:
            raise ValueError("Require dim divisible by heads, head_dim divisible by 8, and even freq_dim.")
        self.dim, self.ffn_dim, self.num_heads = dim, ffn_dim, num_heads
        self.freq_dim, self.latent_channels = freq_dim, latent_channels
        self.gradient_checkpointing = gradient_checkpointing
        checkpointed_layer_indices(num_layers, checkpoint_fraction)
        self.checkpoint_fraction = float(checkpoint_fraction)
        self.activation_offload = bool(activation_offload)
        self.offload_context: Callable = activation_cpu_offload
        self.video_embedder = nn.Linear(latent_channels, dim)
        self.text_embedder = TextProjection(text_dim, dim, ffn_dim, num_heads)
        self.rope = RoPE(dim // num_heads, rope_base)
        self.time_embedding = nn.Sequential(nn.Linear(freq_dim, dim), nn.SiLU(), nn.Linear(dim, dim))
        self.shared_block_modulation = nn.Linear(dim, 6 * dim)
        self.layers = nn.ModuleList([Block(dim, ffn_dim, num_heads, mlp) for _ in range(num_layers)])
        self.final_norm_video = RMSNorm(dim)
        self.final_linear_video = nn.Linear(dim, latent_channels, bias=False)
        self.video_head_modulation = nn.Linear(dim, 2 * dim)

    @property
    def compute_dtype(self) -> torch.dtype:
        return _linear_dtype(self.video_embedder)

    def _time_conditions(self, timestep, batch, device):
        times = torch.as_tensor(timestep, device=device, dtype=torch.float32).reshape(-1).expand(batch)
        half = self.freq_dim // 2
        frequencies = 10000 ** (-torch.arange(half, device=device, dtype=torch.float64) / half)
        phase = times.double()[:, None] * frequencies
        embedding = torch.cat((phase.cos(), phase.sin()), -1).float()
        time = self.time_embedding(embedding.to(_linear_dtype(self.time_embedding[0]))).float()
        modulation = self.shared_block_modulation(time.to(_linear_dtype(self.shared_block_modulation)))
        head = self.video_head_modulation(time.to(_linear_dtype(self.video_head_modulation)))
        return modulation.view(batch, 6, -1), head.view(batch, 2, -1)

    def forward(self, hidden_states, timestep, encoder_hidden_states, encoder_attention_mask=None, skip_layers=None):
        batch = hidden_states.shape[0]
        skipped = frozenset(skip_layers or ())
        mask = encoder_attention_mask
        if mask is None:
            mask = torch.ones(encoder_hidden_states.shape[:2], dtype=torch.bool, device=hidden_states.device)
        outputs = []
        with self.offload_context(self, self.activation_offload, hidden_states.device):
            modulation, head = self._time_conditions(timestep, batch, hidden_states.device)
            for index in range(batch):
                context = encoder_hidden_states[index : index + 1, mask[index].bool()]
                outputs.append(
                    self._forward_sample(
                        hidden_states[index : index + 1], context, modulation[index : index + 1],
                        head[index : index + 1], skipped,
                    )
                )
        return torch.cat(outputs)

    def _project_video(self, latents):
        tokens = latents.flatten(2).transpose(1, 2)
        return self.video_embedder(tokens.to(_linear_dtype(self.video_embedder)).contiguous())

    def _forward_sample(self, hidden_states, context, modulation, head, skipped=frozenset()):
        _, _, height, width = hidden_states.shape
        video = self._project_video(hidden_states)
        rope = self.rope([(0, height, width)], context.shape[1], hidden_states.device).to(video.dtype)
        text = self.text_embedder(context, rope[:, video.shape[1] :])
        tokens = torch.cat((video, text), 1)
        if self.training and not tokens.requires_grad:
            tokens.requires_grad_(True)
        tokens = self._run_layers(tokens, rope, modulation, skipped=skipped)
        predicted = self.final_norm_video(tokens[:, : height * width].to(self.final_norm_video.weight.dtype))
        predicted = predicted * (1 + head[:, 1, None]) + head[:, 0, None]
        predicted = self.final_linear_video(predicted.to(_linear_dtype(self.final_linear_video)))
        return predicted.transpose(1, 2).reshape(1, -1, height, width)

    def forward_packed(self, hidden_states, timestep, encoder_hidden_states):
        """One traversal over concatenated samples (reference model.py:502-626)."""

        batch = len(hidden_states)
        device = hidden_states[0].device
        with self.offload_context(self, self.activation_offload, device):
            modulation, head = self._time_conditions(timestep, batch, device)
            videos, ropes, text_ropes, text_lengths, shapes, joint_lengths = [], [], [], [], [], []
            for target, context in zip(hidden_states, encoder_hidden_states):
                height, width = target.shape[-2:]
                shapes.append((height, width))
                video = self._project_video(target.unsqueeze(0))
                sample_rope = self.rope([(0, height, width)], context.shape[0], device).to(video.dtype)
                videos.append(video)
                ropes.append(sample_rope)
                text_ropes.append(sample_rope[:, video.shape[1] :])
                text_lengths.append(context.shape[0])
                joint_lengths.append(video.shape[1] + context.shape[0])
            text_cu = _cumulative_lengths(text_lengths, device)
            packed_text = torch.cat([context.unsqueeze(0) for context in encoder_hidden_states], 1)
            packed_text = self.text_embedder(packed_text, torch.cat(text_ropes, 1), text_cu)
            text_parts = list(packed_text.split(text_lengths, dim=1))
            tokens = torch.cat([torch.cat((v, t), 1) for v, t in zip(videos, text_parts)], 1)
            rope = torch.cat(ropes, 1)
            if self.training and not tokens.requires_grad:
                tokens.requires_grad_(True)
            tokens = self._run_layers(tokens, rope, modulation, _cumulative_lengths(joint_lengths, device))
            outputs, offset = [], 0
            for index, ((height, width), joint) in enumerate(zip(shapes, joint_lengths)):
                predicted = tokens[:, offset : offset + height * width]
                predicted = self.final_norm_video(predicted.to(self.final_norm_video.weight.dtype))
                predicted = predicted * (1 + head[index : index + 1, 1, None]) + head[index : index + 1, 0, None]
                predicted = self.final_linear_video(predicted.to(_linear_dtype(self.final_linear_video)))
                outputs.append(predicted.transpose(1, 2).reshape(-1, height, width))
                offset += joint
            return outputs

    def _run_layers(self, tokens, rope, modulation, cu_seqlens=None, skipped=frozenset()):
        """Joint blocks with swapping and selective checkpointing (reference model.py:672-710).

        Blocks from ``len(layers) - blocks_to_swap`` on are swapped (``moss_offload.memory``):
        streamed through ``block_swap_manager`` with the next block in traversal order
        prefetched (forward: the following block; recomputation in backward: the preceding
        one), or run from the CPU with ``offloaded_block`` in synchronous mode.
        """

        boundary = len(self.layers) - getattr(self, "blocks_to_swap", 0)
        manager = getattr(self, "block_swap_manager", None)
        streamed = [index for index in range(boundary, len(self.layers)) if index not in skipped]
        position = {index: p for p, index in enumerate(streamed)}
        checkpointed = checkpointed_layer_indices(len(self.layers), self.checkpoint_fraction)
        for index, layer in enumerate(self.layers):
            if index in skipped:
                continue
            # packed: cu_seqlens (a saved tensor, as in the reference) and its lengths as host
            # integers, which a checkpoint keeps as they are (no tensor to offload and restore)
            inputs = (tokens, rope, modulation) if cu_seqlens is None else \
                (tokens, rope, modulation, cu_seqlens, getattr(cu_seqlens, "host_lengths", None))
            if manager is not None and index >= boundary:
                p = position[index]
                tokens = manager.block(
                    index,
                    *inputs,
                    forward_prefetch=streamed[p + 1] if p + 1 < len(streamed) else None,
                    backward_prefetch=streamed[p - 1] if p else None,
                    checkpoint_block=torch.is_grad_enabled(),
                )
            elif index >= boundary:
                from .memory import offloaded_block

                tokens = offloaded_block(layer, *inputs)
            elif self.gradient_checkpointing and self.training and index in checkpointed:
                tokens = checkpoint(layer, *inputs, use_reentrant=False)
            else:
                tokens = layer(*inputs)
        return tokens


# ---------------------------------------------------------------------------------------------
# LoRA (reference lora.py:21-172) and the int8 weight-only base (quantization.py:23-162)


class LoRALinear(nn.Module):
    """Frozen base linear plus ``(alpha / rank) * B @ A``; autocast casts A and B (lora.py:60-86)."""

    def __init__(self, base: nn.Module, rank: int, alpha: float) -> None:
        super().__init__()
        self.base = base
        self.rank = rank
        self.scale = float(alpha) / rank
        self.lora_A = nn.Parameter(torch.empty(rank, base.in_features))
        self.lora_B = nn.Parameter(torch.zeros(base.out_features, rank))
        nn.init.kaiming_uniform_(self.lora_A, a=math.sqrt(5))
        for parameter in self.base.parameters():
            parameter.requires_grad_(False)

    @property
    def compute_dtype(self) -> torch.dtype:
        return _linear_dtype(self.base)

    @property
    def in_features(self):
        return self.base.in_features

    def forward(self, tokens):
        result = self.base(tokens)
        dtype = torch.get_autocast_dtype(tokens.device.type) if torch.is_autocast_enabled(tokens.device.type) else None
        if dtype is None:
            adapter_input, adapter_a, adapter_b = tokens.to(self.lora_A.dtype), self.lora_A, self.lora_B
        else:
            adapter_input, adapter_a, adapter_b = tokens.to(dtype), self.lora_A.to(dtype), self.lora_B.to(dtype)
        update = F.linear(F.linear(adapter_input, adapter_a), adapter_b)
        return result + update.to(result.dtype) * self.scale


class _FrozenInt8Function(torch.autograd.Function):
    """Weight-only int8 linear; saves the int8 weight and fp32 scales (quantization.py:27-65).

    ``backend``: ``hip`` runs the gfx950 MFMA kernels of ``moss_offload.quant_kernels`` (the
    reference's ``triton`` backend), ``eager`` decodes the weight and calls ``F.linear``,
    ``auto`` picks ``hip`` whenever the call is supported.
    """

    @staticmethod
    def forward(ctx, tokens, weight, scale, dtype, backend):
        from . import quant_kernels

        ctx.save_for_backward(weight, scale)
        ctx.input_dtype, ctx.weight_dtype = tokens.dtype, dtype
        ctx.input_shape = tokens.shape
        prepared = tokens.to(dtype)
        selected = quant_kernels.resolve_backend(backend, prepared, weight, scale, dtype)
        if selected == "hip" and torch.is_autocast_enabled(tokens.device.type):
            if torch.get_autocast_dtype(tokens.device.type) != dtype:
                selected = "eager" if backend == "auto" else selected
        ctx.backend = selected
        if selected == "hip":
            result = quant_kernels.int8_linear_forward(prepared, weight, scale)
        else:
            result = F.linear(prepared, quant_kernels.decode(weight, scale, dtype))
        ctx.compute_dtype = result.dtype
        return result

    @staticmethod
    def backward(ctx, gradient):
        from . import quant_kernels

        weight, scale = ctx.saved_tensors
        if ctx.backend == "hip":
            grad = quant_kernels.int8_linear_backward(gradient, weight, scale, ctx.input_shape).to(ctx.input_dtype)
            return grad, None, None, None, None
        with torch.autocast(device_type=gradient.device.type, enabled=False):
            decoded = quant_kernels.decode(weight, scale, ctx.weight_dtype).to(ctx.compute_dtype)
            grad = gradient.to(ctx.compute_dtype).matmul(decoded).to(ctx.input_dtype)
        return grad, None, None, None, None


class FrozenInt8Linear(nn.Module):
    """Per-output-channel symmetric int8 weights, fp32 scales, no bias (quantization.py:68-131)."""

    def __init__(self, weight_int8: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype, backend: str = "auto") -> None:
        super().__init__()
        self.out_features, self.in_features = weight_int8.shape
        self.quantized_backend = backend
        self.register_buffer("weight_int8", weight_int8)
        self.register_buffer("weight_scale", scale.float())
        self.register_buffer("_dtype_anchor", torch.empty(0, device=weight_int8.device, dtype=dtype), persistent=False)

    @property
    def compute_dtype(self):
        return self._dtype_anchor.dtype

    def _apply(self, fn, recurse=True):
        # scales stay fp32 when the model is cast (quantization.py:113-118)
        scale = self.weight_scale
        result = super()._apply(fn, recurse=recurse)
        self.weight_scale = scale.to(device=self.weight_int8.device, dtype=torch.float32)
        return result

    def forward(self, tokens):
        return _FrozenInt8Function.apply(tokens, self.weight_int8, self.weight_scale, self.compute_dtype,
                                         self.quantized_backend)


def configure_quantized_backend(model: nn.Module, backend: str) -> list[str]:
    """Set the backend of every frozen int8 module; return their names (quantization.py:134-144)."""

    from .quant_kernels import BACKENDS

    if backend not in BACKENDS:
        raise ValueError("quantized backend must be auto, eager or hip.")
    names = []
    for name, module in model.named_modules():
        if isinstance(module, FrozenInt8Linear):
            module.quantized_backend = backend
            names.append(name)
    return names


def joint_linear_names(model: MOSSImageTransformer) -> list[str]:
    """Linear modules of the joint blocks, the ``joint`` LoRA target set (lora.py:117-148)."""

    return [
        name
        for name, module in model.named_modules()
        if isinstance(module, (nn.Linear, FrozenInt8Linear)) and name.startswith("layers.")
    ]


def _module_device(module: nn.Module) -> torch.device:
    for tensor in (*module.parameters(), *module.buffers()):
        return tensor.device
    return torch.device("cpu")


def _replace(root: nn.Module, qualified: str, module: nn.Module) -> None:
    parent = root
    parts = qualified.split(".")
    for part in parts[:-1]:
        parent = parent[int(part)] if part.isdigit() else getattr(parent, part)
    if parts[-1].isdigit():
        parent[int(parts[-1])] = module
    else:
        setattr(parent, parts[-1], module)


def inject_lora(model: MOSSImageTransformer, rank: int, alpha: float, b_std: float | None = 0.03) -> list[str]:
    """Freeze the model and wrap the joint-block linears with LoRA (lora.py:151-172).

    ``b_std`` draws ``lora_B ~ N(0, b_std)`` instead of the reference's zeros, so adapter
    gradients are not trivially zero (the reference tests do the same).
    """

    for parameter in model.parameters():
        parameter.requires_grad_(False)
    names = joint_linear_names(model)
    for name in names:
        base = model.get_submodule(name)
        wrapped = LoRALinear(base, rank, alpha).to(device=_module_device(base))
        if b_std is not None:
            with torch.no_grad():
                wrapped.lora_B.normal_(0.0, b_std)
        _replace(model, name, wrapped)
    return names


def quantize_joint_linears(model: MOSSImageTransformer, generator: torch.Generator | None = None) -> list[str]:
    """Replace joint-block linears by int8 weight-only modules with U(0.001, 0.02) scales.

    Synthetic weights: int8 uniform in [-127, 127], per-output-channel scales drawn in fp16
    and stored fp32 (quantization.py:86-91, :116-121 keep scales fp32).
    """

    names = [name for name in joint_linear_names(model) if isinstance(model.get_submodule(name), nn.Linear)]
    for name in names:
        base = model.get_submodule(name)
        device, dtype = base.weight.device, base.weight.dtype
        out_features, in_features = base.weight.shape
        weight = torch.randint(-127, 128, (out_features, in_features), dtype=torch.int8, device=device, generator=generator)
        scale = torch.empty(out_features, dtype=torch.float16, device=device).uniform_(0.001, 0.02, generator=generator)
        _replace(model, name, FrozenInt8Linear(weight, scale.float(), dtype))
    return names


def init_weights(model: nn.Module, std: float = 0.02) -> None:
    """Linear weights ~ N(0, std) in ``named_parameters`` order, biases 0, norm scales 1."""

    with torch.no_grad():
        for name, parameter in model.named_parameters():
            if name.endswith("lora_A.weight") or "lora_" in name:
                continue
            if parameter.dim() >= 2:
                parameter.normal_(0.0, std)
            elif name.endswith("bias"):
                parameter.zero_()
            else:
                parameter.fill_(1.0)


# ---------------------------------------------------------------------------------------------
# flow-matching loss (flow.py:105-135, train.py:102-157)


def noisy_latent(clean, sigma, noise):
    view = sigma.to(clean.dtype).view(-1, *([1] * (clean.ndim - 1)))
    return view * noise + (1 - view) * clean, noise - clean


def squared_error(model, clean, noise, sigma, context, total=1000.0):
    """Sum of squared velocity residuals and the element count for one shape group."""

    noisy, velocity = noisy_latent(clean, sigma, noise)
    prediction = model(noisy.to(model.compute_dtype), sigma.float() * total, context.to(model.compute_dtype))
    residual = prediction.float().sub(velocity.float())
    return residual.square().sum(), residual.numel()
