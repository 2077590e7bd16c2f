"""End-to-end generation over the paged path vs a dense recompute of the same tokens by
the same model: a self-consistency check of the generators' bookkeeping (slots, tables,
positions, chunk boundaries, graph replays).  The comparison with an independent float64
model is tests/test_gpu_model_layers.py's teacher forcing.

Both generators are checked: prefill-first (padded prefill batches, then a graph
decode step) and mixed (chunked prefill and decodes packed into the same steps).

The Generator (nano_inference_amd/e2e.py) prefills prompts through the KV write
and the causal prefill kernel, then decodes token by token through the paged
decode kernel.  Teacher forcing pins it: running the whole sequence (prompt +
generated tokens) through the same model once more, with no metadata (the
layer's dense causal path, src/nano_inference/layers/attention.py:230-231),
must reproduce every greedy choice: at each generated position the chosen
token's logit is the row maximum up to bf16 noise (2e-2 relative to the logit
scale).
"""
import pytest
import torch

from nano_inference_amd import e2e

pytestmark = pytest.mark.gpu


def tiny_config():
    return e2e.Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                           num_heads=4, num_kv_heads=2, head_dim=128, num_layers=2)


def check_teacher_forcing(gen, prompts, new):
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


@pytest.mark.parametrize("prefill_batch", [1, 3])
def test_generation_matches_dense_recompute(prefill_batch):
    cfg = tiny_config()
    prompts = e2e.generation_prompts(5, 3, 70, cfg.vocab_size, seed=11)
    new = 7
    gen = e2e.build(cfg, prompts, max_new_tokens=new, max_prefill_batch=prefill_batch, seed=5)
    st = gen.run(prompts)
    assert st.generated_tokens == len(prompts) * new
    assert st.prefill_steps == -(-len(prompts) // prefill_batch)
    assert st.decode_steps == new - 1
    check_teacher_forcing(gen, prompts, new)


@pytest.mark.parametrize("step_tokens,chunk", [(48, 16), (4096, 512), (7, 3)])
def test_mixed_generation_matches_dense_recompute(step_tokens, chunk):
    """Chunked prefill mixed with decodes (packed steps): the chunks attend through
    the paged cache, decode rows through the decode kernel, in the same steps."""
    cfg = tiny_config()
    prompts = e2e.generation_prompts(6, 3, 90, cfg.vocab_size, seed=12)
    new = 7
    gen = e2e.build(cfg, prompts, max_new_tokens=new, seed=5, mixed=True,
                    max_step_tokens=step_tokens, chunk=chunk)
    free0 = len(gen.pool.free)
    st = gen.run(prompts)
    assert st.generated_tokens == len(prompts) * new
    assert len(gen.pool.free) == free0
    check_teacher_forcing(gen, prompts, new)


def test_kv_pool_blocks_are_returned():
    cfg = tiny_config()
    prompts = e2e.generation_prompts(3, 10, 40, cfg.vocab_size, seed=3)
    gen = e2e.build(cfg, prompts, max_new_tokens=3, max_prefill_batch=2, seed=1)
    free0 = len(gen.pool.free)
    gen.run(prompts)
    assert len(gen.pool.free) == free0


def test_graph_decode_reproduces_eager_decode():
    """The captured decode step, replayed with eager work and a sync between replays,
    yields the eager loop's tokens exactly (same kernels, same order)."""
    cfg = tiny_config()
    prompts = e2e.generation_prompts(6, 5, 90, cfg.vocab_size, seed=21)
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


def test_mixed_graph_tail_reproduces_eager_tail():
    """The mixed generator's captured decode tail, replayed with eager work and a
    sync between replays, yields the eager tail's tokens exactly."""
    cfg = tiny_config()
    prompts = e2e.generation_prompts(6, 5, 90, cfg.vocab_size, seed=22)
    kw = dict(max_new_tokens=9, seed=9, mixed=True, max_step_tokens=40, chunk=16)
    eager = e2e.build(cfg, prompts, use_graph=False, **kw)
    eager.run(prompts)
    graph = e2e.build(cfg, prompts, use_graph=True, **kw)
    scratch = torch.empty(1 << 20, device="cuda")

    def between():
        scratch.normal_()
        torch.cuda.synchronize()

    graph.replay_hook = between
    graph.run(prompts)
    assert graph.outputs == eager.outputs
    check_teacher_forcing(graph, prompts, 9)


@pytest.mark.parametrize("mixed", [False, True])
def test_generation_with_fp8_cache(mixed):
    """Both generators over an fp8 KV pool.  The prefill-first generator's first token
    comes from attention over the fresh K/V, so it equals the bf16 pool's exactly; the
    rest read the fp8 cache (its parity is checked at the layer and kernel level)."""
    cfg = tiny_config()
    prompts = e2e.generation_prompts(5, 3, 70, cfg.vocab_size, seed=13)
    kw = dict(max_new_tokens=6, seed=5, mixed=mixed, max_step_tokens=48, chunk=16)
    ref_gen = e2e.build(cfg, prompts, **kw)
    ref_gen.run(prompts)
    gen = e2e.build(cfg, prompts, fp8_cache=True, **kw)
    assert gen.pool.k_cache.dtype == torch.uint8
    free0 = len(gen.pool.free)
    st = gen.run(prompts)
    assert st.generated_tokens == len(prompts) * 6
    assert len(gen.pool.free) == free0
    for out, ref_out in zip(gen.outputs, ref_gen.outputs):
        assert len(out) == 6 and all(0 <= t < cfg.vocab_size for t in out)
        if not mixed:
            assert out[0] == ref_out[0]
