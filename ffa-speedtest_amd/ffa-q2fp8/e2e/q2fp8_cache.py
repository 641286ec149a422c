"""Hugging Face integration of the q2fp8 pruned decode: a paged KV cache and a decode attention hook.

The reference integrates its fp8fp8 kernel into a copied Llama (ffa-fp8fp8/e2e/fp8fp8_cache.py:183-224,
ffa-fp8fp8/e2e/modeling_llama.py:293-321): a `Cache` subclass stores the quantized K, and the attention
forward calls the FFA decode when a step has one query token.  Its cache rebuilds a dequantized copy of
all keys on every update (fp8fp8_cache.py:60-69) and grows by `torch.cat`.

Here, for q2fp8, on the MI355X library:

* `Q2FP8Cache` / `Q2FP8PagedLayer`: every layer keeps a `PagedQ2Cache` (64-token pages, g32 2-bit codes +
  fp8 residual K, V^T pages) sized once for `max_batch_size` x `max_cache_len`, with a seeded page table.
  `update()` g32-quantizes and appends the new (already rotated) K and V in one kernel
  (`ffa_q2_quantize_g32_append`) and never dequantizes the cache.
* `ffa_q2fp8_attention`: registered with transformers' attention registry as "ffa_q2fp8", so an
  unmodified `LlamaForCausalLM` (or any model whose attention goes through `ALL_ATTENTION_FUNCTIONS`)
  uses it once `enable_ffa_q2fp8(model, ...)` is called.  As in the reference's hook
  (modeling_llama.py:281-337, settings from `config.attn_settings`, e2e/bench_llama_fp8fp8.py:179-189):
  a step with one query token per sequence, `use_ffa_decode` set and the layer in `pattern_layers`
  (default: every layer) runs the pruned decode over the paged cache (BS, SBS, delta,
  use_fp8_residual); every other step -- the prompt, a later multi-token chunk, decode steps of layers
  outside `pattern_layers` or with `use_ffa_decode=False` -- runs exact causal attention over the
  cache's own keys and values dequantized by `ffa_q2_paged_dequant` (the reference attends with
  FlashAttention to the keys its cache returns dequantized from every update, fp8fp8_cache.py:60-69,
  84-89).  The exact attention itself is fp32 torch matmuls, as the reference's is a library call.

The HF models apply RoPE (their half-split `rotate_half`) before `Cache.update`, so the cache receives
rotated K and appends it with the quantize-append entry point; the fused K-projection + RoPE producer
follows the reference producer's interleaved-pair RoPE instead and serves the benchmark path.

Limits: all sequences of a batch have the same length (no padding), no beam search reordering.
"""
from __future__ import annotations

import math
import sys
import threading
from pathlib import Path
from typing import Any, Callable, Optional

import torch
from transformers import AttentionInterface
from transformers.cache_utils import Cache, CacheLayerMixin

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))  # ffa-speedtest_amd/
from ffa_mi355x.decode import DecodeWorkspace  # noqa: E402
from ffa_mi355x.paged import PAGE, PagedQ2Cache  # noqa: E402

__all__ = ["Q2FP8Cache", "Q2FP8PagedLayer", "ffa_q2fp8_attention", "enable_ffa_q2fp8"]

ATTN_NAME = "ffa_q2fp8"
DEFAULT_SETTINGS = dict(use_ffa_decode=True, BS=64, SBS=64, delta=5.0, use_fp8_residual=True, pattern_layers=None)
# (layer index, layer) of the update() that ran last on this thread; the attention of that layer
# takes it (and clears it), so a model run without a Q2FP8Cache cannot pick up a stale layer
_current = threading.local()


class Q2FP8PagedLayer(CacheLayerMixin):
    """One layer's paged q2fp8 cache (pools allocated on the first update)."""

    is_sliding = False

    def __init__(self, max_batch_size: int, max_cache_len: int, res_dtype=torch.float8_e4m3fn, page_seed: int = 0):
        super().__init__()
        self.max_batch_size = int(max_batch_size)
        self.max_cache_len = int(max_cache_len)
        self.res_dtype = res_dtype
        self.page_seed = page_seed
        self.pool: Optional[PagedQ2Cache] = None
        self.block_table: Optional[torch.Tensor] = None
        self.seq_lens: Optional[torch.Tensor] = None
        self.seq_len = 0
        self._workspace: Optional[DecodeWorkspace] = None

    @property
    def capacity(self) -> int:
        return self.block_table.shape[1] * PAGE

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        B, HKV, _, D = key_states.shape
        if D != 128:
            raise NotImplementedError(f"head_dim {D}: the q2fp8 decode implements 128")
        if B > self.max_batch_size:
            raise ValueError(f"batch {B} exceeds max_batch_size {self.max_batch_size}")
        self.dtype, self.device = key_states.dtype, key_states.device
        npg = -(-self.max_cache_len // PAGE)
        # V pages hold fp16(V): the decode's P.V operand, converted once per token at append
        self.pool = PagedQ2Cache(B * npg, HKV, self.device, res_dtype=self.res_dtype, v_dtype=torch.float16)
        # a seeded permutation of the pool: sequences' pages are scattered as in a serving cache
        perm = torch.randperm(B * npg, generator=torch.Generator().manual_seed(self.page_seed))
        self.block_table = perm.view(B, npg).to(torch.int32).to(self.device)
        self.seq_lens = torch.zeros(B, dtype=torch.int32, device=self.device)
        self.seq_len = 0
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Append K / V [B, HKV, Tn, 128] (rotated) at the current length; returns them unchanged."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        B, HKV, Tn, D = key_states.shape
        if B != self.block_table.shape[0] or HKV != self.pool.HKV:
            raise ValueError("key_states do not match the cache's batch / KV heads")
        if self.seq_len + Tn > self.capacity:
            raise ValueError(f"cache holds {self.capacity} tokens, {self.seq_len + Tn} requested")
        pos = torch.full((B,), self.seq_len, dtype=torch.int32, device=self.device)
        self.pool.append(key_states.transpose(1, 2).contiguous(), value_states.transpose(1, 2).contiguous(), pos,
                         self.block_table)
        self.seq_len += Tn
        self.seq_lens.fill_(self.seq_len)
        self.last_query_len = Tn
        return key_states, value_states

    def workspace(self, HQ: int, BS: int, SBS: int, dtype) -> DecodeWorkspace:
        B = self.block_table.shape[0]
        ws = self._workspace
        if ws is None or not ws.matches(B, HQ, self.pool.HKV, self.capacity, BS, SBS, self.device, dtype):
            ws = self._workspace = DecodeWorkspace(B, HQ, self.pool.HKV, self.capacity, BS, SBS, self.device, dtype)
        return ws

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.seq_len + query_length, 0

    def get_seq_length(self) -> int:
        return self.seq_len

    def get_max_length(self) -> int:
        return self.max_cache_len

    def reset(self) -> None:
        self.seq_len = 0
        if self.seq_lens is not None:
            self.seq_lens.zero_()

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        raise NotImplementedError("beam search reordering is not supported by the paged q2fp8 cache")

    def offload(self):
        raise NotImplementedError("offloading is not supported by the paged q2fp8 cache")

    def prefetch(self):
        pass


class Q2FP8Cache(Cache):
    """Paged q2fp8 KV cache for a whole model (one Q2FP8PagedLayer per decoder layer)."""

    def __init__(self, num_layers: int, max_batch_size: int, max_cache_len: int, res_dtype=torch.float8_e4m3fn,
                 page_seed: int = 0):
        layers = [Q2FP8PagedLayer(max_batch_size, max_cache_len, res_dtype, page_seed + i) for i in range(num_layers)]
        super().__init__(layers=layers)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args, **kwargs):
        out = self.layers[layer_idx].update(key_states, value_states)
        _current.entry = (layer_idx, self.layers[layer_idx])  # taken by ffa_q2fp8_attention of that layer
        return out


def exact_attention(query: torch.Tensor, layer: Q2FP8PagedLayer, scaling: float) -> torch.Tensor:
    """Causal attention of the L newest query tokens [B, HQ, L, D] over the whole cache (positions
    seq_len - L .. seq_len - 1 see the keys up to their own position), on the keys and values the
    cache holds, dequantized in the model dtype (fp32 arithmetic, contiguous operands).  Returns
    [B, L, HQ, D]."""
    B, HQ, L, D = query.shape
    S = layer.seq_len
    k, v = layer.pool.dequantize(layer.block_table, S, layer.seq_lens, out_dtype=layer.dtype)
    G = HQ // layer.pool.HKV
    k = k[:, :S].float().transpose(1, 2).repeat_interleave(G, dim=1).contiguous()  # [B, HQ, S, D]
    v = v[:, :S].float().transpose(1, 2).repeat_interleave(G, dim=1).contiguous()
    s = torch.matmul(query.float().contiguous(), k.transpose(2, 3).contiguous()) * scaling
    qpos = torch.arange(S - L, S, device=s.device)[:, None]
    s = s.masked_fill(torch.arange(S, device=s.device)[None, :] > qpos, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v).to(query.dtype).transpose(1, 2).contiguous()


def ffa_q2fp8_attention(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, attention_mask,
                        scaling: Optional[float] = None, dropout: float = 0.0, **kwargs):
    """Attention of one layer (the transformers attention-function signature); query [B, HQ, L, D] rotated.

    L == 1 with use_ffa_decode and the layer in pattern_layers: the pruned q2fp8 decode over the
    layer's paged cache (modeling_llama.py:293-321's branch); otherwise exact causal attention over
    the cache's dequantized keys and values (:322-337)."""
    settings = dict(DEFAULT_SETTINGS)
    settings.update(getattr(module.config, "attn_settings", None) or {})
    entry = getattr(_current, "entry", None)
    _current.entry = None
    if entry is None or not isinstance(entry[1], Q2FP8PagedLayer):
        raise RuntimeError("ffa_q2fp8 attention needs a Q2FP8Cache passed as past_key_values (with use_cache)")
    layer_idx, layer = entry
    if getattr(module, "layer_idx", layer_idx) != layer_idx:
        raise RuntimeError(f"ffa_q2fp8 attention of layer {module.layer_idx} after the cache update of layer "
                           f"{layer_idx}")
    B, HQ, L, D = query.shape
    scale = scaling if scaling is not None else 1.0 / math.sqrt(D)
    pattern = settings.get("pattern_layers")
    if pattern is not None and not isinstance(pattern, (list, tuple)):
        raise TypeError("pattern_layers must be a list of layer indices")
    if L == 1 and settings["use_ffa_decode"] and (pattern is None or layer_idx in pattern):
        ws = layer.workspace(HQ, settings["BS"], settings["SBS"], query.dtype)
        layer.pool.decode(query[:, :, 0, :].contiguous(), layer.block_table, layer.seq_lens, T=layer.capacity,
                          scale=scale, BS=settings["BS"], SBS=settings["SBS"], delta=settings["delta"],
                          use_fp8_residual=settings["use_fp8_residual"], workspace=ws)
        out = ws.o.unsqueeze(1)  # [B, 1, HQ, D]
        hook: Optional[Callable] = settings.get("on_decode")
        if hook is not None:
            hook(layer_idx, query[:, :, 0, :], out[:, 0], layer)
        return out, None
    out = exact_attention(query, layer, scale)
    hook = settings.get("on_exact")
    if hook is not None:
        hook(layer_idx, query, out, layer)
    return out, None


def enable_ffa_q2fp8(model, **attn_settings: Any) -> None:
    """Route the model's attention through ffa_q2fp8_attention (registered once) with these settings
    (BS, SBS, delta, use_fp8_residual, use_ffa_decode, pattern_layers; optional
    on_decode(layer_idx, q, o, cache_layer) and on_exact(layer_idx, q, o, cache_layer) observers)."""
    AttentionInterface.register(ATTN_NAME, ffa_q2fp8_attention)
    cfg = model.config
    cfg.attn_settings = {**DEFAULT_SETTINGS, **attn_settings}
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation(ATTN_NAME)
    else:
        cfg._attn_implementation = ATTN_NAME
