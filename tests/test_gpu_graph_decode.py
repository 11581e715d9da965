"""Graph-replayed decode steps (CapturedDecode) against eager steps.

A patched transformers MistralForCausalLM (random fp16 weights; 2 layers,
8 query / 2 KV heads of dim 128, or 32 / 8 for the branch-free decode
kernel) runs a 600-token prompt (one cold block
plus an 88-token tail per layer) for one or two sequences, then 12
teacher-forced one-token steps three ways from the same cache state:
  * CapturedDecode: one eager warm-up step, one capture, ten replays, with
    eager work (argmax, a copy) and a synchronisation between replays;
  * eager steps with the same pinned decode grid: every step's logits must be
    bit-identical to the replayed ones (same kernels, same launch shapes,
    device counters advanced by the replays themselves);
  * eager steps with the grid the host mirror gives (unpinned): equal up to
    the fp16 rounding of a different block split.
The caches' counters and host mirrors must agree after the segment."""
import pytest
import torch

pytestmark = pytest.mark.gpu

VOCAB = 512


def _model(seed=5, heads=(8, 2)):
    from transformers import MistralConfig, MistralForCausalLM
    cfg = MistralConfig(vocab_size=VOCAB, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                        num_attention_heads=heads[0], num_key_value_heads=heads[1], head_dim=128,
                        max_position_embeddings=4096, rope_theta=1e6, sliding_window=None)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    return MistralForCausalLM(cfg).eval().to(device="cuda", dtype=torch.float16)


def _snapshot(model):
    return [layer.self_attn._spectral_cache.clone() for layer in model.model.layers]


def _restore(model, caches):
    for layer, c in zip(model.model.layers, caches):
        layer.self_attn._spectral_cache = c.clone()


@pytest.mark.parametrize("batch,heads", [(1, (8, 2)), (2, (8, 2)), (2, (32, 8))])
@torch.no_grad()
def test_captured_decode_replays_match_eager_steps(batch, heads):
    from unsloth_spectral import CapturedDecode, _lib, patch_unsloth_attention
    model = _model(heads=heads)   # 32/8 heads: the branch-free decode kernel of the model loop
    n_prompt, steps = 600, 12
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, VOCAB, (batch, n_prompt + steps), generator=g).cuda()
    patch_unsloth_attention(model, use_triton_kernel=True, verbose=False)
    model(input_ids=ids[:, :n_prompt], use_cache=False, logits_to_keep=1)
    snap = _snapshot(model)
    tail0 = [c.hot_len for c in snap]
    assert all(c.num_cold_blocks == 1 for c in snap) and tail0 == [n_prompt - 512] * 2

    def token(i):
        return ids[:, n_prompt + i]

    def position(i):
        return torch.full((batch, 1), n_prompt + i, dtype=torch.long, device="cuda")

    # graph-replayed segment
    dec = CapturedDecode(model, steps)
    graph_logits = []
    for i in range(steps):
        lg = dec.step(token(i), position(i))
        graph_logits.append(lg.float().clone())
        torch.cuda.synchronize()
        _ = lg.argmax(-1).clone()                    # eager work between replays
    assert dec.graph is not None and dec.left == 0
    after = [layer.self_attn._spectral_cache for layer in model.model.layers]
    for c in after:
        assert c._grid_tail is None
        assert c.hot_len == n_prompt - 512 + steps and c.current_position == n_prompt + steps
        assert c.counters[:, _lib.SC_CNT_TAIL_LEN].tolist() == [c.hot_len] * batch  # device = host mirror
    graph_logits = torch.stack(graph_logits)

    # eager steps, same pinned grid, from the same cache state
    _restore(model, snap)
    for layer in model.model.layers:
        c = layer.self_attn._spectral_cache
        c._grid_tail = c.hot_len + steps
    pinned = torch.stack([model(input_ids=token(i)[:, None], position_ids=position(i), use_cache=False,
                                logits_to_keep=1).logits[:, -1].float() for i in range(steps)])
    for layer in model.model.layers:
        layer.self_attn._spectral_cache._grid_tail = None
    assert torch.equal(graph_logits, pinned), (graph_logits - pinned).abs().max().item()

    # eager steps with the host mirror's grid
    _restore(model, snap)
    plain = torch.stack([model(input_ids=token(i)[:, None], position_ids=position(i), use_cache=False,
                               logits_to_keep=1).logits[:, -1].float() for i in range(steps)])
    err = ((graph_logits - plain).abs().max() / plain.abs().max()).item()
    print(f"replayed vs unpinned eager: max |dlogit| / max |logit| = {err:.2e}")
    assert err < 1e-2


def test_captured_decode_refuses_a_block_boundary():
    from unsloth_spectral import CapturedDecode, patch_unsloth_attention
    model = _model()
    ids = torch.randint(0, VOCAB, (1, 500), generator=torch.Generator().manual_seed(7)).cuda()
    patch_unsloth_attention(model, verbose=False)
    with torch.no_grad():
        model(input_ids=ids, use_cache=False, logits_to_keep=1)
    with pytest.raises(ValueError, match="block boundary"):
        CapturedDecode(model, 20)                    # tail 500 + 20 crosses 512
