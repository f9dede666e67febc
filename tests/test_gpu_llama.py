"""The drop-in shim end to end on a small random-weight Llama (transformers'
own LlamaForCausalLM, 2 layers, 8 query / 2 KV heads, head_dim 64): one
chunked-prefill forward then one decode step through pagedattn.llama, against
the same model in fp32 on the CPU over the whole sequences (eager attention).
Logits agree within bf16 tolerance; the fused launches (RoPE + append, RoPE + append + decode)
give exactly the logits of the separate reference calls."""

import copy

import numpy as np
import pytest
import torch

from pagedattn import llama as L
from pagedattn.capacity import new_kv_scales
from pagedattn.metadata import decode_metadata, prefill_metadata

from paged_cases import i32, random_tables

pytestmark = pytest.mark.gpu


def _tiny_llama():
    """fp32 CPU reference model (its attention stays off the GPU)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=512, intermediate_size=1024, num_attention_heads=8,
                      num_key_value_heads=2, num_hidden_layers=2, vocab_size=512,
                      max_position_embeddings=4096, attn_implementation="eager")
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


def _run_paged(model, device, tokens, lens, tables, num_pages, fuse, kv_dtype=torch.bfloat16):
    cfg = model.config
    hkv, d = cfg.num_key_value_heads, cfg.hidden_size // cfg.num_attention_heads
    shape = (cfg.num_hidden_layers, num_pages, 2, hkv, 16, d)
    if kv_dtype == torch.float8_e4m3fn:
        pool = torch.zeros(shape, dtype=torch.uint8, device=device).view(kv_dtype)
    else:
        pool = torch.zeros(shape, dtype=kv_dtype, device=device)
    L.FUSE = fuse
    scales = new_kv_scales(pool) if kv_dtype == torch.float8_e4m3fn else None
    L.init_flashinfer_state(kv_pool=pool, page_size=16, device=device, kv_scales=scales,
                            kv_scale_policy="running")
    # prefill: every sequence's first lens[b] tokens in one packed forward
    meta = prefill_metadata(tables, [0] * len(lens), lens)
    L.build_batch_indices_positions(i32(meta.qo_indptr, device), i32(meta.seq_lens, device))
    L.plan_prefill(qo_indptr=i32(meta.qo_indptr, device), kv_indptr=i32(meta.kv_indptr, device),
                   kv_indices=i32(meta.kv_indices, device),
                   kv_last_page_len=i32(meta.kv_last_page_len, device),
                   num_qo_heads=cfg.num_attention_heads, num_kv_heads=hkv, head_dim=d)
    packed = torch.cat([tokens[b, :n] for b, n in enumerate(lens)])[None]
    with torch.no_grad():
        pre = model(input_ids=packed, use_cache=False).logits[0]
    ends = np.cumsum(lens) - 1
    pre_last = pre[torch.as_tensor(ends, device=device)]
    # decode: token lens[b] of every sequence
    new_lens = [n + 1 for n in lens]
    meta = decode_metadata(tables, new_lens)
    L.FlashInferState.batch_indices = i32(meta.batch_indices, device)
    L.FlashInferState.positions = i32(meta.positions, device)
    L.plan_decode(kv_indptr=i32(meta.kv_indptr, device), kv_indices=i32(meta.kv_indices, device),
                  kv_last_page_len=i32(meta.kv_last_page_len, device),
                  num_qo_heads=cfg.num_attention_heads, num_kv_heads=hkv, head_dim=d)
    step = torch.stack([tokens[b, n] for b, n in enumerate(lens)])[:, None]
    with torch.no_grad():
        dec = model(input_ids=step, use_cache=False).logits[:, 0]
    return pre_last.float(), dec.float(), scales


def test_patched_llama_matches_eager_model(gpu):
    ref = _tiny_llama()
    model = copy.deepcopy(ref).to(device=gpu, dtype=torch.bfloat16)
    L.patch_llama_model(model)
    lens = [37, 100, 5, 64]
    rng = np.random.default_rng(0)
    tokens = torch.as_tensor(rng.integers(0, ref.config.vocab_size, size=(len(lens), 128)))
    tokens_gpu = tokens.to(gpu)
    tables, num_pages = random_tables(rng, [n + 1 for n in lens], extra_pages=4)
    fused = _run_paged(model, gpu, tokens_gpu, lens, tables, num_pages, fuse=True)
    plain = _run_paged(model, gpu, tokens_gpu, lens, tables, num_pages, fuse=False)
    L.FUSE = True
    # the fused launches reproduce the separate calls exactly
    assert torch.equal(fused[0], plain[0])
    assert torch.equal(fused[1], plain[1])
    # and both follow the model's own attention over the whole sequence
    _check_against_model(ref, tokens, lens, fused, 3e-2)


def _check_against_model(ref, tokens, lens, got_logits, tol):
    with torch.no_grad():
        for b, n in enumerate(lens):
            full = ref(input_ids=tokens[b:b + 1, :n + 1], use_cache=False).logits[0].float()
            for got, want in ((got_logits[0][b], full[n - 1]), (got_logits[1][b], full[n])):
                got = got.cpu()
                rel = float((got - want).norm() / want.norm())
                assert rel < tol, (b, rel)


def test_patched_llama_e4m3_pool_running_scales(gpu):
    """An e4m3 pool written by the engine itself: every append keeps its
    pages' scales a running amax (powers of two)."""
    ref = _tiny_llama()
    model = copy.deepcopy(ref).to(device=gpu, dtype=torch.bfloat16)
    L.patch_llama_model(model)
    lens = [37, 100, 5, 64]
    rng = np.random.default_rng(1)
    tokens = torch.as_tensor(rng.integers(0, ref.config.vocab_size, size=(len(lens), 128)))
    tables, num_pages = random_tables(rng, [n + 1 for n in lens], extra_pages=4)
    out = _run_paged(model, gpu, tokens.to(gpu), lens, tables, num_pages, fuse=True,
                     kv_dtype=torch.float8_e4m3fn)
    used = sorted({p for t in tables for p in t})
    sc = out[2][:, used].cpu()
    assert bool((sc > 0).all())
    assert bool((torch.frexp(sc).mantissa == 0.5).all())
    _check_against_model(ref, tokens, lens, out, 8e-2)
