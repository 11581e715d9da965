"""patch_unsloth_attention on a transformers MistralForCausalLM (random
weights; 2 layers, 8 query / 2 KV heads of dim 128, theta 1e6, fp16).

The patched model is stepped the way generation steps it: one prefill call
over the prompt, then one-token calls with explicit position ids (teacher
forced with fixed tokens, so both sides see the same inputs).  Each layer
appends the pre-RoPE K/V to its own SpectralCache (compression fires inside
the append) and then attends (integration.py:596-659).

  * No cold block in the context: the spectral path holds the exact FP16
    keys, so the logits of the patched model (fp32 weights and activations,
    fp16 attention) must equal the unpatched fp32 model's (run on the CPU)
    within the noise of the fp16 attention.
  * Cold blocks, with a block boundary crossed during decode: the logits of
    the HIP prefill and decode kernels must equal those of dense attention
    over the cache's own reconstruction (use_spectral_attention=False, which
    is the reference's dense path over get_kv, integration.py:292-402).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

VOCAB = 512


def _model(seed=0):
    """fp32 model on the CPU (the unpatched reference runs there); the
    caller moves it to the GPU in fp16."""
    from transformers import MistralConfig, MistralForCausalLM
    cfg = MistralConfig(vocab_size=VOCAB, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                        num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                        max_position_embeddings=4096, rope_theta=1e6, sliding_window=None)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    model = MistralForCausalLM(cfg).eval()
    with torch.no_grad():  # larger Q/K weights: peaked attention, so position errors show
        for layer in model.model.layers:
            layer.self_attn.q_proj.weight.mul_(4.0)
            layer.self_attn.k_proj.weight.mul_(4.0)
    return model


def _gpu(model, dtype=torch.float16):
    return model.to(device="cuda", dtype=dtype)


def _tokens(n, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, VOCAB, (1, n), generator=g)


@torch.no_grad()
def _run_patched(model, ids, n_prompt):
    """Prefill over ids[:, :n_prompt], then one call per remaining token;
    returns the logits that predict tokens n_prompt .. len-1 ([steps+1, V])."""
    out = [model(input_ids=ids[:, :n_prompt], use_cache=False).logits[0, -1].float()]
    for p in range(n_prompt, ids.shape[1] - 1):
        pos = torch.tensor([[p]], device=ids.device)
        out.append(model(input_ids=ids[:, p:p + 1], position_ids=pos, use_cache=False).logits[0, -1].float())
    return torch.stack(out)


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


def _same_choice(a, b):
    """Greedy choices agree wherever the reference's top-2 gap exceeds twice
    the largest logit difference (closer calls may flip on FP16 noise)."""
    top2 = b.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * (a - b).abs().max()
    return torch.equal(a.argmax(-1)[clear], b.argmax(-1)[clear])


@pytest.mark.parametrize("absolute", [True, False])
def test_tail_only_context_matches_unpatched_model(absolute):
    from unsloth_spectral import get_cache_stats, patch_unsloth_attention
    model = _model()
    n_prompt, steps = 200, 12
    ids = _tokens(n_prompt + steps)
    with torch.no_grad():                         # unpatched model, fp32, CPU
        ref = model(input_ids=ids, use_cache=False).logits[0, n_prompt - 1:-1].float().cuda()
    model = _gpu(model, torch.float32)  # fp32 around attention: only the fp16 attention path differs
    patch_unsloth_attention(model, use_triton_kernel=absolute, verbose=False)
    got = _run_patched(model, ids.cuda(), n_prompt)
    assert got.shape == ref.shape
    err = _rel(got, ref)
    print(f"absolute={absolute}: max |dlogit| / max |logit| = {err:.2e}")
    assert err < 5e-3
    assert _same_choice(got, ref)
    st = get_cache_stats(model)
    assert st["layers_with_cache"] == 2 and st["total_blocks"] == 0
    assert st["total_tokens"] == 2 * (n_prompt + steps - 1)


def test_cold_blocks_and_decode_compression_match_dense_over_tiers():
    from unsloth_spectral import get_cache_stats, patch_unsloth_attention
    from unsloth_spectral.integration import reset_spectral_caches
    model = _gpu(_model(seed=3))
    n_prompt, steps = 1020, 10     # prefill leaves 1 cold block + 508 tail; token 1024 compresses
    ids = _tokens(n_prompt + steps, seed=4).cuda()
    patch_unsloth_attention(model, verbose=False)
    kernel = _run_patched(model, ids, n_prompt)
    st = get_cache_stats(model)
    caches = [layer.self_attn._spectral_cache for layer in model.model.layers]
    assert st["total_blocks"] == 2 * 2
    assert all(c.num_cold_blocks == 2 and c.hot_len == n_prompt + steps - 1 - 1024 for c in caches)
    assert all(c.current_position == n_prompt + steps - 1 for c in caches)

    reset_spectral_caches(model)
    patch_unsloth_attention(model, use_spectral_attention=False, verbose=False)
    dense = _run_patched(model, ids, n_prompt)
    err0 = _rel(kernel[:1], dense[:1])             # prefill: HIP prefill kernel vs dense over get_kv
    print(f"prefill kernel vs dense over the reconstruction: {err0:.2e}")
    assert err0 < 1e-2
    err = _rel(kernel, dense)
    print(f"decode kernel vs dense over the reconstruction: {err:.2e}")
    assert err < 1e-2
    assert _same_choice(kernel, dense)


def test_left_padded_batch_generation_matches_unpatched_model():
    """Batched greedy generation with a left-padded prompt (HF generate):
    the pad keys enter the cache but are never attended (the prompt's mask
    is kept as the cache's key mask), so the patched model's logits equal
    the unpatched model's (fp32 weights, fp16 attention on our side)."""
    from unsloth_spectral import patch_unsloth_attention
    model = _model(seed=5)
    n = 60
    ids = _tokens(2 * n, seed=6).reshape(2, n)
    am = torch.ones(2, n, dtype=torch.long)
    am[0, :7] = 0                                   # sequence 0: 7 pad tokens on the left
    ref_model = _gpu(model, torch.float32)
    with torch.no_grad():
        ref = ref_model.generate(ids.cuda(), attention_mask=am.cuda(), max_new_tokens=8, do_sample=False,
                                 output_logits=True, return_dict_in_generate=True, pad_token_id=0)
    ref_logits = torch.stack(ref.logits, 1).float()            # [2, 8, V]
    patch_unsloth_attention(ref_model, verbose=False)
    with torch.no_grad():
        got = ref_model.generate(ids.cuda(), attention_mask=am.cuda(), max_new_tokens=8, do_sample=False,
                                 output_logits=True, return_dict_in_generate=True, pad_token_id=0)
    got_logits = torch.stack(got.logits, 1).float()
    for b in range(2):
        # the two runs feed back their own greedy tokens: compare the steps
        # up to the first differing token (identical inputs until then),
        # and accept a differing token only where the reference's top two
        # logits are closer than twice the logit error
        same = (got.sequences[b, n:] == ref.sequences[b, n:]).tolist()
        upto = same.index(False) + 1 if False in same else len(same)
        err = _rel(got_logits[b, :upto], ref_logits[b, :upto])
        print(f"sequence {b}: {upto} steps with equal inputs, max |dlogit| / max |logit| = {err:.2e}")
        assert err < 5e-3, b
        assert _same_choice(got_logits[b, :upto], ref_logits[b, :upto])
        assert upto >= 4, b
    cache = ref_model.model.layers[0].self_attn._spectral_cache
    assert cache.key_mask is not None and int(cache.key_mask[0, :7].sum()) == 0


def test_decode_steps_of_the_patched_attention_do_not_synchronise():
    """After the prompt (through the whole model), one-token steps through a
    patched attention module -- the call transformers makes per layer, with
    position ids on the device and a block compressed on the way -- run
    under torch's sync debug mode "error": no step waits for the device.
    (transformers' own mask preparation around the layers reads the device
    on its own, e.g. masking_utils.eager_mask builds a scalar tensor on the
    device, so the check is made at the attention module.)"""
    from unsloth_spectral import patch_unsloth_attention
    model = _gpu(_model(seed=7))
    patch_unsloth_attention(model, block_size=128, verbose=False)
    n_prompt, steps = 120, 12                       # the block boundary at 128 is crossed during decode
    ids = _tokens(n_prompt, seed=8).cuda()
    attn = model.model.layers[0].self_attn
    rotary = model.model.rotary_emb
    pos_all = torch.arange(n_prompt + steps, device="cuda")[None]
    g = torch.Generator(device="cuda").manual_seed(9)
    hidden = torch.randn(steps, 1, 1, model.config.hidden_size, generator=g, device="cuda").half()
    with torch.no_grad():
        model(input_ids=ids, position_ids=pos_all[:, :n_prompt], use_cache=False)
        cos, sin = rotary(hidden[0], pos_all)                  # [1, L, D] tables of the positions
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            for i in range(steps):
                p = n_prompt + i
                out, _ = attn(hidden[i], position_embeddings=(cos[:, p:p + 1], sin[:, p:p + 1]),
                              attention_mask=None, position_ids=pos_all[:, p:p + 1])
        finally:
            torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    cache = attn._spectral_cache
    assert cache.num_cold_blocks == 1 and cache.total_tokens == n_prompt + steps
    assert torch.isfinite(out).all()
