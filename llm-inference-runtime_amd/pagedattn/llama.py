"""Drop-in counterpart of the serving engine's attention shim
(src/models/llama.py:1-382) running on the gfx950 paged-attention module.

The engine imports exactly these names (src/engine/async_engine.py:21,
src/engine/runtime/step_executor.py:8-13): ``FlashInferState``,
``init_flashinfer_state``, ``build_batch_indices_positions``,
``plan_prefill``, ``plan_decode`` and ``patch_llama_model``; the patched
``LlamaAttention.forward`` keeps the reference's op order
(qkv projection -> split -> RoPE -> page append -> attention -> o_proj).

Deliberate differences from the reference:
* RoPE theta/scaling are read from ``config.rope_parameters`` when present
  (transformers >= 5 moved them there; the reference's
  ``getattr(config, "rope_theta", 10000.0)`` at src/models/llama.py:346
  silently falls back to 10000 for Llama-3).
* bitsandbytes 4-bit projections (src/models/llama.py:283-336) are not fused
  (bitsandbytes is CUDA-only); such a model raises NotImplementedError.
* The pool may be e4m3 with ``FlashInferState.kv_scales`` [L, P, 2, Hkv].
  With ``kv_scale_policy == "running"`` (the default) every append keeps
  the scales of the pages it writes a running amax
  (``append_paged_kv_cache_e4m3_amax``); ``"fixed"`` encodes with the scales
  as given (pools quantised ahead of time).
"""

from __future__ import annotations

from typing import cast

import torch
from torch import nn

from . import ops


# Fused launches on the engine's hot path: RoPE + append (+ decode attention)
# in one kernel each.  False runs the three reference calls separately.
FUSE = True


class FlashInferState:
    """Process-global state shared by all layers of one forward
    (src/models/llama.py:16-36).  Attributes are writable from outside: the
    decode step writes ``batch_indices``/``positions`` directly
    (src/engine/runtime/step_executor.py:220-225)."""

    kv_pool: torch.Tensor | None = None
    kv_scales: torch.Tensor | None = None  # e4m3 pools only: [L, P, 2, Hkv]
    kv_scale_policy: str = "running"  # e4m3 pools: "running" amax or "fixed" scales

    kv_indices: torch.Tensor | None = None
    kv_indptr: torch.Tensor | None = None
    kv_last_page_len: torch.Tensor | None = None

    batch_indices: torch.Tensor | None = None
    positions: torch.Tensor | None = None

    workspace_buffer: torch.Tensor | None = None

    prefill_wrapper: ops.BatchPrefillWithPagedKVCacheWrapper | None = None
    decode_wrapper: ops.BatchDecodeWithPagedKVCacheWrapper | None = None

    page_size: int = 16
    dtype: torch.dtype | None = None

    mode: str = "prefill"

    # set by plan_decode: (batch_indices tensor, its version) when the step's
    # token rows are sequences 0..B-1 in order, which the fused decode launch
    # requires; None otherwise
    _fused_rows: tuple | None = None


WORKSPACE_BYTES = 128 * 1024 * 1024


def init_flashinfer_state(*, kv_pool: torch.Tensor, page_size: int, device,
                          kv_scales: torch.Tensor | None = None,
                          kv_scale_policy: str = "running") -> None:
    """Store the pool, allocate the 128 MiB workspace and the two wrappers
    (src/models/llama.py:39-67)."""
    if page_size != ops.PAGE_SIZE:
        raise NotImplementedError(f"page_size {page_size} (only 16 is implemented)")
    if kv_scale_policy not in ("running", "fixed"):
        raise ValueError(f"kv_scale_policy {kv_scale_policy!r}: 'running' or 'fixed'")
    FlashInferState.kv_pool = kv_pool
    FlashInferState.kv_scales = kv_scales
    FlashInferState.kv_scale_policy = kv_scale_policy
    FlashInferState.page_size = page_size
    FlashInferState.dtype = kv_pool.dtype
    ws = torch.zeros(WORKSPACE_BYTES, dtype=torch.uint8, device=device)
    FlashInferState.workspace_buffer = ws
    FlashInferState.prefill_wrapper = ops.BatchPrefillWithPagedKVCacheWrapper(ws, "HND")
    FlashInferState.decode_wrapper = ops.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")


def append_error_count() -> int:
    """Tokens the page appends skipped since init because their metadata
    pointed outside the page table (reads the device counter: synchronises).
    Every append path, the fused decode launches included, counts into the
    int32 at byte 0 of the workspace."""
    ws = FlashInferState.workspace_buffer
    if ws is None:
        return 0
    return int(ws[:4].view(torch.int32)[0].item())


def append_clamp_count() -> int:
    """8-element pieces of rows written to an e4m3 pool with fixed scales
    that were clamped at +-448 (or met a bad scale) since init (synchronises;
    the int32 at byte 4 of the workspace).  Kept apart from
    append_error_count(): clamps are routine with scales taken from earlier
    rows, skipped tokens are not."""
    ws = FlashInferState.workspace_buffer
    if ws is None:
        return 0
    return int(ws[4:8].view(torch.int32)[0].item())


def build_batch_indices_positions(append_indptr: torch.Tensor, seq_lens: torch.Tensor,
                                  nnz: int | None = None) -> None:
    """(src/models/llama.py:70-83).  The token count comes from `nnz` when
    the caller knows it (the rows of its q, or the token capacity it gave
    build_paged_metadata, which fills qo_indptr on the device): then nothing
    is copied to the host.  Otherwise it is read from append_indptr[-1] as
    the reference does -- without a sync when append_indptr lives on the
    host, with one device-to-host copy when it lives on the GPU."""
    if nnz is None:
        nnz = int(append_indptr[-1].item())
    FlashInferState.batch_indices, FlashInferState.positions = ops.get_batch_indices_positions(
        append_indptr, seq_lens, nnz)


def _q_dtype() -> torch.dtype:
    dt = FlashInferState.dtype
    # an e4m3 pool still runs bf16 queries
    return torch.bfloat16 if dt == torch.float8_e4m3fn else cast(torch.dtype, dt)


def plan_prefill(*, qo_indptr: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                 kv_last_page_len: torch.Tensor, num_qo_heads: int, num_kv_heads: int,
                 head_dim: int, max_qo_tokens: int | None = None) -> None:
    """(src/models/llama.py:86-116).  With max_qo_tokens (a bound on the
    step's query tokens) the plan is made on the device by every run: the
    metadata tensors are read in place and nothing is copied to the host, as
    a step captured in a HIP graph needs."""
    FlashInferState.mode = "prefill"
    FlashInferState.kv_indptr = kv_indptr
    FlashInferState.kv_indices = kv_indices
    FlashInferState.kv_last_page_len = kv_last_page_len
    pw = cast(ops.BatchPrefillWithPagedKVCacheWrapper, FlashInferState.prefill_wrapper)
    pw.begin_forward(qo_indptr, kv_indptr, kv_indices, kv_last_page_len, num_qo_heads,
                     num_kv_heads, head_dim, FlashInferState.page_size, q_data_type=_q_dtype(),
                     device_plan=max_qo_tokens is not None, max_qo_tokens=max_qo_tokens)


def plan_decode(*, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                kv_last_page_len: torch.Tensor, num_qo_heads: int, num_kv_heads: int,
                head_dim: int) -> None:
    """(src/models/llama.py:119-147).  The planner needs kv_indptr and
    kv_last_page_len on the host; batch_indices travels in the same
    device-to-host copy, so the check for the fused decode rows costs no
    transfer of its own."""
    FlashInferState.mode = "decode"
    FlashInferState.kv_indptr = kv_indptr
    FlashInferState.kv_indices = kv_indices
    FlashInferState.kv_last_page_len = kv_last_page_len
    bsz = kv_last_page_len.numel()
    bi = FlashInferState.batch_indices
    check = (bi is not None and bi.numel() == bsz and bi.device == kv_indptr.device
             and kv_last_page_len.device == kv_indptr.device)
    parts = [kv_indptr.reshape(-1).to(torch.int32), kv_last_page_len.reshape(-1).to(torch.int32)]
    if check:
        parts.append(cast(torch.Tensor, bi).detach().reshape(-1).to(torch.int32))
    if kv_last_page_len.device == kv_indptr.device:
        host = torch.cat(parts).cpu()
    else:
        host = torch.cat([p.cpu() for p in parts])
    n_ptr = kv_indptr.numel()
    indptr_h, last_h = host[:n_ptr], host[n_ptr:n_ptr + bsz]
    dw = cast(ops.BatchDecodeWithPagedKVCacheWrapper, FlashInferState.decode_wrapper)
    dw.begin_forward(kv_indptr, kv_indices, kv_last_page_len, num_qo_heads, num_kv_heads,
                     head_dim, FlashInferState.page_size, q_data_type=_q_dtype(),
                     indptr_host=indptr_h.reshape(kv_indptr.shape),
                     last_page_len_host=last_h.reshape(kv_last_page_len.shape))
    FlashInferState._fused_rows = (
        _identity_rows(cast(torch.Tensor, bi), host[n_ptr + bsz:]) if check else None)


def _identity_rows(batch_indices: torch.Tensor, host_rows: torch.Tensor) -> tuple | None:
    """(batch_indices, its in-place version) when its host copy `host_rows`
    is arange(B), the engine's decode rows (step_executor.py:220-222), else
    None."""
    if not torch.equal(host_rows.to(torch.int64), torch.arange(host_rows.numel(), dtype=torch.int64)):
        return None
    return batch_indices, batch_indices._version


def patched_llama_attention_forward(self, hidden_states: torch.Tensor,
                                    position_embeddings=None, attention_mask=None,
                                    past_key_value=None, output_attentions=False,
                                    use_cache=False, cache_position=None, **kwargs):
    """LlamaAttention.forward over the paged pool (src/models/llama.py:150-249).
    Extra decoder kwargs (position_ids, past_key_values, ...) are ignored: the
    positions come from FlashInferState."""
    bsz, q_len, _ = hidden_states.shape
    qkv = self.qkv_proj(hidden_states)
    q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
    q_rows = q.view(-1, self.num_heads, self.head_dim)
    k_rows = k.view(-1, self.num_key_value_heads, self.head_dim)
    v_rows = v.view(-1, self.num_key_value_heads, self.head_dim)

    positions = cast(torch.Tensor, FlashInferState.positions)
    pool = cast(torch.Tensor, FlashInferState.kv_pool)
    layer_pool = pool[self.layer_idx]
    scales = FlashInferState.kv_scales
    layer_scales = scales[self.layer_idx] if scales is not None else None
    ws = cast(torch.Tensor, FlashInferState.workspace_buffer)
    decode = FlashInferState.mode != "prefill"
    running = (layer_scales is not None and pool.dtype == torch.float8_e4m3fn
               and FlashInferState.kv_scale_policy == "running")

    if running:
        # e4m3 pages whose scales follow the rows written: RoPE, then the
        # running-amax append (its scale updates are not fused into attention)
        ops.apply_rope_pos_ids_inplace(q_rows, k_rows, positions, rope_theta=self.rope_theta,
                                       rope_scale=self.rope_scale, interleave=False)
        ops.append_paged_kv_cache_e4m3_amax(
            k_rows, v_rows, cast(torch.Tensor, FlashInferState.batch_indices), positions,
            layer_pool, cast(torch.Tensor, FlashInferState.kv_indices),
            cast(torch.Tensor, FlashInferState.kv_indptr),
            cast(torch.Tensor, FlashInferState.kv_last_page_len), layer_scales,
            kv_layout="HND", error_flag=ws[:8].view(torch.int32))
    elif FUSE and decode and _decode_rows_match(q_rows):
        # RoPE + append + attention of the decode step in one launch
        dw = cast(ops.BatchDecodeWithPagedKVCacheWrapper, FlashInferState.decode_wrapper)
        out = dw.run(q_rows, layer_pool, kv_scales=layer_scales, append_key=k_rows,
                     append_value=v_rows, rope=(self.rope_scale, self.rope_theta),
                     positions=positions)
        return self.o_proj(out.reshape(bsz, 1, self.num_heads * self.head_dim)), None
    elif FUSE:
        # RoPE + append in one launch, then attention
        ops.rope_append_paged_kv_cache(
            q_rows, k_rows, v_rows, cast(torch.Tensor, FlashInferState.batch_indices),
            positions, layer_pool, cast(torch.Tensor, FlashInferState.kv_indices),
            cast(torch.Tensor, FlashInferState.kv_indptr),
            cast(torch.Tensor, FlashInferState.kv_last_page_len), kv_layout="HND",
            rope_scale=self.rope_scale, rope_theta=self.rope_theta, kv_scales=layer_scales,
            error_flag=ws[:8].view(torch.int32))
    else:
        ops.apply_rope_pos_ids_inplace(q_rows, k_rows, positions, rope_theta=self.rope_theta,
                                       rope_scale=self.rope_scale, interleave=False)
        ops.append_paged_kv_cache(
            k_rows, v_rows, cast(torch.Tensor, FlashInferState.batch_indices), positions,
            layer_pool, cast(torch.Tensor, FlashInferState.kv_indices),
            cast(torch.Tensor, FlashInferState.kv_indptr),
            cast(torch.Tensor, FlashInferState.kv_last_page_len), kv_layout="HND",
            kv_scales=layer_scales, error_flag=ws[:8].view(torch.int32))

    if not decode:
        pw = cast(ops.BatchPrefillWithPagedKVCacheWrapper, FlashInferState.prefill_wrapper)
        out = pw.forward(q_rows, layer_pool, causal=True, kv_scales=layer_scales)
        out = out.reshape(bsz, q_len, self.num_heads * self.head_dim)
    else:
        dw = cast(ops.BatchDecodeWithPagedKVCacheWrapper, FlashInferState.decode_wrapper)
        out = dw.forward(q_rows, layer_pool, kv_scales=layer_scales)
        out = out.reshape(bsz, 1, self.num_heads * self.head_dim)
    return self.o_proj(out), None


def _decode_rows_match(q_rows: torch.Tensor) -> bool:
    """The fused decode launch appends row b to sequence b: it applies when
    the step carries exactly one new token per planned sequence in sequence
    order, i.e. the batch_indices that plan_decode saw were arange(B) and
    that tensor is still the state's, unmodified (the engine's decode step,
    step_executor.py:204-234).  Otherwise the separate RoPE + append and
    attention launches run, which honour any batch_indices."""
    dw = cast(ops.BatchDecodeWithPagedKVCacheWrapper, FlashInferState.decode_wrapper)
    rec = FlashInferState._fused_rows
    bi = FlashInferState.batch_indices
    return (rec is not None and rec[0] is bi and bi._version == rec[1]
            and q_rows.shape[0] == getattr(dw, "_bsz", -1))


def _fuse_qkv_proj(attn) -> nn.Linear:
    """One Linear whose output rows are q | k | v (src/models/llama.py:256-280)."""
    parts = [attn.q_proj, attn.k_proj, attn.v_proj]
    for p in parts:
        if not isinstance(p, nn.Linear):
            raise NotImplementedError(
                f"{type(p).__name__} projections (e.g. bitsandbytes 4-bit) are not supported")
    has_bias = any(p.bias is not None for p in parts)
    w0 = attn.q_proj.weight
    fused = nn.Linear(w0.shape[1], sum(p.weight.shape[0] for p in parts), bias=has_bias,
                      device=w0.device, dtype=w0.dtype)
    with torch.no_grad():
        fused.weight.copy_(torch.cat([p.weight for p in parts], dim=0))
        if has_bias:
            fused.bias.copy_(torch.cat([
                p.bias if p.bias is not None else torch.zeros(p.weight.shape[0], dtype=w0.dtype,
                                                              device=w0.device)
                for p in parts]))
    return fused


def rope_config(config) -> tuple[float, float]:
    """(rope_theta, linear rope_scale) of a Llama config; rejects scaling
    types that a single linear factor cannot express (src/models/llama.py:346-361)."""
    params = getattr(config, "rope_parameters", None)
    if isinstance(params, dict) and params:
        theta = float(params.get("rope_theta", getattr(config, "rope_theta", 10000.0)))
        scaling = params
    else:
        theta = float(getattr(config, "rope_theta", 10000.0))
        scaling = getattr(config, "rope_scaling", None)
    scale = 1.0
    if scaling:
        rope_type = scaling.get("rope_type", scaling.get("type"))
        if rope_type not in (None, "default", "linear"):
            raise NotImplementedError(
                f"rope scaling type {rope_type!r} is not a linear position scale")
        if rope_type == "linear":
            scale = float(scaling.get("factor", 1.0))
    return theta, scale


def patch_llama_model(model) -> None:
    """Install the paged forward on every decoder layer (src/models/llama.py:345-382)."""
    from transformers.models.llama.modeling_llama import LlamaAttention

    cfg = model.config
    theta, scale = rope_config(cfg)
    for idx, layer in enumerate(model.model.layers):
        attn = layer.self_attn
        attn.layer_idx = idx
        attn.num_heads = cfg.num_attention_heads
        attn.num_key_value_heads = cfg.num_key_value_heads
        attn.head_dim = cfg.hidden_size // cfg.num_attention_heads
        attn.q_size = attn.num_heads * attn.head_dim
        attn.kv_size = attn.num_key_value_heads * attn.head_dim
        attn.rope_theta = theta
        attn.rope_scale = scale
        attn.qkv_proj = _fuse_qkv_proj(attn)
        del attn.q_proj, attn.k_proj, attn.v_proj
        attn.forward = patched_llama_attention_forward.__get__(attn, LlamaAttention)
