"""End-to-end generation over the paged path vs a dense recompute of the same tokens.

The Generator (nano_inference_amd/e2e.py) prefills prompts through the KV write
and the causal prefill kernel, then decodes token by token through the paged
decode kernel.  Teacher forcing pins it: running the whole sequence (prompt +
generated tokens) through the same model once more, with no metadata (the
layer's dense causal path, src/nano_inference/layers/attention.py:230-231),
must reproduce every greedy choice: at each generated position the chosen
token's logit is the row maximum up to bf16 noise (2e-2 relative to the logit
scale), and the logits of the last position agree with the incremental path's.
"""
import pytest
import torch

from nano_inference_amd import e2e

pytestmark = pytest.mark.gpu


def tiny_config():
    return e2e.Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                           num_heads=4, num_kv_heads=2, head_dim=128, num_layers=2)


@pytest.mark.parametrize("prefill_batch", [1, 3])
def test_generation_matches_dense_recompute(prefill_batch):
    cfg = tiny_config()
    prompts = e2e.config4_prompts(5, 3, 70, cfg.vocab_size, seed=11)
    new = 7
    gen = e2e.build(cfg, prompts, max_new_tokens=new, max_prefill_batch=prefill_batch, seed=5)
    st = gen.run(prompts)
    assert st.generated_tokens == len(prompts) * new
    assert st.prefill_steps == -(-len(prompts) // prefill_batch)
    assert st.decode_steps == new - 1
    model = gen.model
    for prompt, out in zip(prompts, gen.outputs):
        assert len(out) == new
        seq = torch.tensor(prompt + out[:-1], device="cuda").unsqueeze(0)
        n = seq.shape[1]
        with torch.no_grad():
            x = model.embed_tokens(seq)
            pos = torch.arange(n, device="cuda").unsqueeze(0)
            for layer in model.layers:
                x = layer(x, pos, None, None)
            logits = model.lm_head(model.norm(x[0])).float()
        scale = logits.abs().max().item()
        for i, tok in enumerate(out):
            row = logits[len(prompt) - 1 + i]
            assert row.max().item() - row[tok].item() <= 2e-2 * scale, (
                f"position {i}: chose {tok}, dense argmax {row.argmax().item()}")


def test_kv_pool_blocks_are_returned():
    cfg = tiny_config()
    prompts = e2e.config4_prompts(3, 10, 40, cfg.vocab_size, seed=3)
    gen = e2e.build(cfg, prompts, max_new_tokens=3, max_prefill_batch=2, seed=1)
    free0 = len(gen.pool.free)
    gen.run(prompts)
    assert len(gen.pool.free) == free0


def test_graph_decode_reproduces_eager_decode():
    """The captured decode step, replayed with eager work and a sync between replays,
    yields the eager loop's tokens exactly (same kernels, same order)."""
    cfg = tiny_config()
    prompts = e2e.config4_prompts(6, 5, 90, cfg.vocab_size, seed=21)
    eager = e2e.build(cfg, prompts, max_new_tokens=9, max_prefill_batch=4, seed=9)
    eager.run(prompts)
    graph = e2e.build(cfg, prompts, max_new_tokens=9, max_prefill_batch=4, seed=9,
                      use_graph=True)
    scratch = torch.empty(1 << 20, device="cuda")

    def between():
        scratch.normal_()
        torch.cuda.synchronize()

    graph.replay_hook = between
    st = graph.run(prompts)
    assert st.decode_steps == 8
    assert graph.outputs == eager.outputs
