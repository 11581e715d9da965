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
