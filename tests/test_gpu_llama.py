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


def _run_paged(model, device, tokens, lens, tables, num_pages, fuse, kv_dtype=torch.bfloat16,
               perm=None):
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
    bi, pos = meta.batch_indices, meta.positions
    if perm is not None:
        # token row j is appended to sequence perm[j] (at its new position)
        bi = np.asarray(perm, np.int32)
        pos = meta.positions[bi]
    L.FlashInferState.batch_indices = i32(bi, device)
    L.FlashInferState.positions = i32(pos, device)
    L.plan_decode(kv_indptr=i32(meta.kv_indptr, device), kv_indices=i32(meta.kv_indices, device),
                  kv_last_page_len=i32(meta.kv_last_page_len, device),
                  num_qo_heads=cfg.num_attention_heads, num_kv_heads=hkv, head_dim=d)
    step = torch.stack([tokens[b, n] for b, n in enumerate(lens)])[:, None]
    with torch.no_grad():
        dec = model(input_ids=step, use_cache=False).logits[:, 0]
    return pre_last.float(), dec.float(), scales, L.FlashInferState.kv_pool.clone()


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


def test_fused_decode_needs_identity_rows(gpu):
    """A decode step whose batch_indices is not arange(B) (the state is
    writable, step_executor.py:220-225) must not take the fused launch, which
    appends row b to sequence b: with FUSE on, the logits and the pool equal
    those of the separate RoPE / append / attention calls."""
    ref = _tiny_llama()
    model = copy.deepcopy(ref).to(device=gpu, dtype=torch.bfloat16)
    L.patch_llama_model(model)
    lens = [37, 100, 5, 64]
    rng = np.random.default_rng(2)
    tokens = torch.as_tensor(rng.integers(0, ref.config.vocab_size, size=(len(lens), 128)))
    tables, num_pages = random_tables(rng, [n + 1 for n in lens], extra_pages=4)
    perm = [2, 0, 3, 1]
    fused = _run_paged(model, gpu, tokens.to(gpu), lens, tables, num_pages, fuse=True,
                       perm=perm)
    plain = _run_paged(model, gpu, tokens.to(gpu), lens, tables, num_pages, fuse=False,
                       perm=perm)
    L.FUSE = True
    assert torch.equal(fused[1], plain[1])
    assert torch.equal(fused[3], plain[3])
    # and an identity step does take it (its result differs from the permuted one)
    ident = _run_paged(model, gpu, tokens.to(gpu), lens, tables, num_pages, fuse=True)
    assert not torch.equal(ident[3], fused[3])


def test_plan_decode_one_host_copy(gpu):
    """plan_decode brings kv_indptr, kv_last_page_len and batch_indices to the
    host in one device-to-host copy (the planner needs the first two; the
    third decides whether the fused decode launch applies): torch's sync
    debug mode sees exactly one synchronising operation, and the fused rows
    are still recognised (and rejected for a permutation)."""
    import warnings
    L.init_flashinfer_state(kv_pool=torch.zeros((1, 64, 2, 2, 16, 64), dtype=torch.bfloat16,
                                                device=gpu), page_size=16, device=gpu)
    rng = np.random.default_rng(3)
    lens = [37, 100, 5, 64]
    tables, _ = random_tables(rng, lens, extra_pages=4)
    meta = decode_metadata(tables, lens)
    args = dict(kv_indptr=i32(meta.kv_indptr, gpu), kv_indices=i32(meta.kv_indices, gpu),
                kv_last_page_len=i32(meta.kv_last_page_len, gpu), num_qo_heads=8,
                num_kv_heads=2, head_dim=64)
    for rows, fused in ((np.arange(4), True), (np.array([2, 0, 3, 1]), False)):
        L.FlashInferState.batch_indices = i32(rows.astype(np.int32), gpu)
        torch.cuda.synchronize()
        prev = torch.cuda.get_sync_debug_mode()
        torch.cuda.set_sync_debug_mode("warn")
        try:
            with warnings.catch_warnings(record=True) as caught:
                warnings.simplefilter("always")
                L.plan_decode(**args)
        finally:
            torch.cuda.set_sync_debug_mode(prev)
        syncs = [w for w in caught if "synchroniz" in str(w.message)]
        assert len(syncs) == 1, [str(w.message) for w in syncs]
        assert (L.FlashInferState._fused_rows is not None) == fused


# -----------------------------------------------------------------------------
# "Option A" of the integration: the engine keeps its own attention shim and
# imports this package under FlashInfer's name.  The forward and state set-up
# below issue the FlashInfer calls with the argument forms that shim uses
# (src/models/llama.py:49-67 constructors, :79-83, :106-116 and :138-147
# plans with positional shapes and q_data_type=, :175-182 RoPE with keyword
# theta/scale, :188-210 all-keyword append, :218-222 forward(q=,
# paged_kv_cache=, causal=True), :236-239 forward(q=, paged_kv_cache=)),
# through `pagedattn` itself.

def _flashinfer_form_forward(self, hidden_states, position_embeddings=None,
                             attention_mask=None, past_key_value=None, output_attentions=False,
                             use_cache=False, cache_position=None, **kwargs):
    import pagedattn as flashinfer
    st = L.FlashInferState
    n_seq, q_len, _ = hidden_states.shape
    q, k, v = self.qkv_proj(hidden_states).split([self.q_size, self.kv_size, self.kv_size],
                                                 dim=-1)
    q3 = q.view(-1, self.num_heads, self.head_dim)
    k3 = k.view(-1, self.num_key_value_heads, self.head_dim)
    v3 = v.view(-1, self.num_key_value_heads, self.head_dim)
    flashinfer.apply_rope_pos_ids_inplace(q3, k3, st.positions, rope_theta=self.rope_theta,
                                          rope_scale=self.rope_scale, interleave=False)
    layer = st.kv_pool[self.layer_idx]
    flashinfer.append_paged_kv_cache(append_key=k3, append_value=v3,
                                     batch_indices=st.batch_indices, positions=st.positions,
                                     paged_kv_cache=layer, kv_indices=st.kv_indices,
                                     kv_indptr=st.kv_indptr,
                                     kv_last_page_len=st.kv_last_page_len, kv_layout="HND")
    if st.mode == "prefill":
        o = st.prefill_wrapper.forward(q=q3, paged_kv_cache=layer, causal=True)
        o = o.reshape(n_seq, q_len, self.num_heads * self.head_dim)
    else:
        o = st.decode_wrapper.forward(q=q3, paged_kv_cache=layer)
        o = o.reshape(n_seq, 1, self.num_heads * self.head_dim)
    return self.o_proj(o), None


def _run_flashinfer_form(model, device, tokens, lens, tables, num_pages):
    import pagedattn as flashinfer
    from transformers.models.llama.modeling_llama import LlamaAttention
    cfg = model.config
    hq, hkv = cfg.num_attention_heads, cfg.num_key_value_heads
    d = cfg.hidden_size // hq
    for layer in model.model.layers:
        layer.self_attn.forward = _flashinfer_form_forward.__get__(layer.self_attn,
                                                                   LlamaAttention)
    st = L.FlashInferState
    st.kv_pool = torch.zeros((cfg.num_hidden_layers, num_pages, 2, hkv, 16, d),
                             dtype=torch.bfloat16, device=device)
    st.page_size = 16
    st.dtype = st.kv_pool.dtype
    # an uninitialised workspace, as the engine allocates it (torch.empty)
    st.workspace_buffer = torch.empty(128 * 1024 * 1024, dtype=torch.uint8,
                                      device=device).fill_(0xA5)
    st.prefill_wrapper = flashinfer.BatchPrefillWithPagedKVCacheWrapper(st.workspace_buffer,
                                                                        "HND")
    st.decode_wrapper = flashinfer.BatchDecodeWithPagedKVCacheWrapper(st.workspace_buffer,
                                                                      "HND")
    meta = prefill_metadata(tables, [0] * len(lens), lens)
    qo_indptr = i32(meta.qo_indptr, device)
    nnz = int(qo_indptr[-1].item())
    st.batch_indices, st.positions = flashinfer.get_batch_indices_positions(
        qo_indptr, i32(meta.seq_lens, device), nnz)
    st.mode = "prefill"
    st.kv_indptr, st.kv_indices = i32(meta.kv_indptr, device), i32(meta.kv_indices, device)
    st.kv_last_page_len = i32(meta.kv_last_page_len, device)
    st.prefill_wrapper.begin_forward(qo_indptr, st.kv_indptr, st.kv_indices,
                                     st.kv_last_page_len, hq, hkv, d, st.page_size,
                                     q_data_type=st.dtype)
    packed = torch.cat([tokens[b, :n] for b, n in enumerate(lens)])[None]
    with torch.no_grad():
        pre = model(input_ids=packed, use_cache=False).logits[0]
    pre_last = pre[torch.as_tensor(np.cumsum(lens) - 1, device=device)]
    dm = decode_metadata(tables, [n + 1 for n in lens])
    st.batch_indices = torch.arange(len(lens), dtype=torch.int32, device=device)
    st.positions = i32(dm.positions, device)
    st.mode = "decode"
    st.kv_indptr, st.kv_indices = i32(dm.kv_indptr, device), i32(dm.kv_indices, device)
    st.kv_last_page_len = i32(dm.kv_last_page_len, device)
    st.decode_wrapper.begin_forward(st.kv_indptr, st.kv_indices, st.kv_last_page_len, hq, hkv,
                                    d, st.page_size, q_data_type=st.dtype)
    step = torch.stack([tokens[b, n] for b, n in enumerate(lens)])[:, None]
    with torch.no_grad():
        dec = model(input_ids=step, use_cache=False).logits[:, 0]
    return pre_last.float(), dec.float(), st.kv_pool.clone()


def test_flashinfer_call_forms_through_pagedattn(gpu):
    ref = _tiny_llama()
    lens = [37, 100, 5, 64]
    rng = np.random.default_rng(3)
    tokens = torch.as_tensor(rng.integers(0, ref.config.vocab_size, size=(len(lens), 128)))
    tables, num_pages = random_tables(rng, [n + 1 for n in lens], extra_pages=4)
    m1 = copy.deepcopy(ref).to(device=gpu, dtype=torch.bfloat16)
    L.patch_llama_model(m1)
    shim = _run_paged(m1, gpu, tokens.to(gpu), lens, tables, num_pages, fuse=True)
    m2 = copy.deepcopy(ref).to(device=gpu, dtype=torch.bfloat16)
    L.patch_llama_model(m2)
    opt_a = _run_flashinfer_form(m2, gpu, tokens.to(gpu), lens, tables, num_pages)
    # the separate FlashInfer-named calls equal the shim's fused launches bit for bit
    assert torch.equal(opt_a[0], shim[0])
    assert torch.equal(opt_a[1], shim[1])
    assert torch.equal(opt_a[2], shim[3])
    _check_against_model(ref, tokens, lens, (opt_a[0], opt_a[1]), 3e-2)
