"""Benchmark of the gfx950 attention path (one JSON line on stdout).

Workload (``config.workload``): paged decode at the Qwen3-8B layout - 64
sequences, 32 query / 8 KV heads, head_dim 128, contexts uniform in
[512, 8192], block size 16, a shuffled 40,000-block pool, bf16.  One step is
one attention layer's decode pass: write the 64 new K/V tokens into the cache
(nia_kv_write), then paged decode attention (nia_paged_decode).  Steps rotate
over 4 cache layers so that no step finds the previous step's KV in the
256 MB last-level cache.

value = algorithmic HBM bytes of a step / step time, in GB/s.  The bytes are
  decode:  sum_i L_i * H_kv * D * 2 * 2 (K and V) + 2 * B * H * D * 2 (q, out)
           + 4 * sum_i ceil(L_i / 16) (block table) + 8 * B (context_lens)
  write:   4 * B * H_kv * D * 2 (read k, v; write both caches) + 8 * B (slots)
The JSON line also carries the decode kernel's roofline (HBM, 8 TB/s peak),
causal prefill TFLOP/s against bf16 MFMA peak (2.5 PFLOP/s dense), the other
synthetic workloads, and the reference's CPU attention timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       python bench.py --profile WORKLOAD [--launches N]
           (three 1 GiB copies, then N launches of one workload, for rocprofv3 counter
            runs; WORKLOAD: decode, decode_vl, decode_fp8, kv_write, kv_write_prefill,
            prefill, chunked, vision_full, vision_window)
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
DECODE_LAYERS = 4


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def warm_up(torch, fn, seconds: float = 0.1) -> None:
    """Run fn until `seconds` of wall time have passed.  The GPU raises its clocks over
    the first few milliseconds of sustained work (and lowers them when idle), so every
    measured leg first runs its own work for a while."""
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def time_calls(torch, fn, iters: int, rounds: int = 5) -> float:
    """Milliseconds per call of fn: after a warm-up, `rounds` batches of `iters`
    back-to-back calls are timed with events; the median batch mean is returned."""
    warm_up(torch, fn)
    means = []
    for _ in range(rounds):
        a, b = _events(torch)
        a.record()
        for i in range(iters):
            fn(i)
        b.record()
        torch.cuda.synchronize()
        means.append(a.elapsed_time(b) / iters)
    return sorted(means)[len(means) // 2]


def per_call_ms(torch, fn, iters: int) -> float:
    """Mean of per-call event timings (each call bracketed by its own events)."""
    pairs = []
    for i in range(iters):
        a, b = _events(torch)
        a.record()
        fn(i)
        b.record()
        pairs.append((a, b))
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in pairs) / iters


def graph_call_ms(torch, fn, calls: int = 50, rounds: int = 5) -> float:
    """Device time per call of a short kernel: `calls` calls captured in one HIP graph,
    replayed `rounds` times after a warm-up; median replay time / calls.  (Timed one
    by one, a kernel of a few microseconds measures the host's launch rate instead.)"""
    fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(calls):
            fn(i)
    warm_up(torch, lambda _: g.replay(), 0.05)
    times = []
    for _ in range(rounds):
        a, b = _events(torch)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / calls)
    return sorted(times)[len(times) // 2]


def source_digest(paths) -> str:
    """sha256 of the kernel sources a counter summary was measured on."""
    h = hashlib.sha256()
    for rel in paths:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


DECODE_SOURCES = ("nano-inference_amd/csrc/paged_decode.hip", "nano-inference_amd/csrc/common.h")
KV_WRITE_SOURCES = ("nano-inference_amd/csrc/kv_write.hip", "nano-inference_amd/csrc/common.h")
PREFILL_SOURCES = ("nano-inference_amd/csrc/prefill.hip", "nano-inference_amd/csrc/common.h")


def read_traffic(workload: str, sources=DECODE_SOURCES):
    """Per-launch HBM bytes of a kernel from its committed counter summary
    (profiles/traffic_<workload>.txt), or None when there is none or when it was measured
    on other kernel sources (its source_sha256 line differs from the sources here)."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    vals, digest = {}, None
    with open(path) as f:
        for line in f:
            m = re.match(r"\s*source_sha256\s*[:=]\s*([0-9a-f]{64})", line)
            if m:
                digest = m.group(1)
                continue
            m = re.match(r"\s*(\w+)\s*[:=]\s*([0-9.eE+-]+)", line)
            if m:
                vals[m.group(1)] = float(m.group(2))
    if digest != source_digest(sources):
        return None
    return vals.get("hbm_bytes_per_launch")


def bench_decode(torch, ops, workloads, steps: int, warmup: int):
    c = workloads.decode_qwen3_8b("cuda", layers=DECODE_LAYERS)
    b, h, d = c.q.shape
    out = torch.empty_like(c.q)
    ws = torch.empty(ops.decode_workspace_bytes(b, h, c.num_kv_heads, c.block_tables.shape[1],
                                                16, d), dtype=torch.uint8, device="cuda")

    def write(i):
        L = i % DECODE_LAYERS
        ops.kv_write(c.k_new, c.v_new, c.k_cache[L], c.v_cache[L], c.slot_mapping)

    def decode(i):
        L = i % DECODE_LAYERS
        ops.paged_decode(c.q, c.k_cache[L], c.v_cache[L], c.block_tables, c.context_lens,
                         out=out, workspace=ws)

    def step(i):
        write(i)
        decode(i)

    warm_up(torch, step)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    a, e = _events(torch)
    a.record()
    for i in range(steps):
        step(i)
    e.record()
    torch.cuda.synchronize()
    ms_step = a.elapsed_time(e) / steps
    iters = max(steps, 30)
    # the launch duration: back-to-back calls between two events (what a kernel trace
    # shows per launch); each call between events of its own also counts the event
    # packets' dispatch latency (~5 us), reported beside it
    dec_ms = time_calls(torch, decode, iters)
    dec_bracketed_ms = per_call_ms(torch, decode, iters)
    wr_ms = graph_call_ms(torch, lambda _: write(0))
    return c, ms_step, dec_ms, dec_bracketed_ms, wr_ms


def bench_prefill(torch, ops, workloads):
    res = {}
    c = workloads.prefill_qwen3_8b("cuda")
    cu = c.cu_seqlens
    qs, ql = cu[:-1].contiguous(), (cu[1:] - cu[:-1]).contiguous()
    out = torch.empty_like(c.q)
    mq = max(c.lens)

    def run(_):
        ops.prefill(c.q, c.k, c.v, qs, ql, qs, ql, mq, ops.CAUSAL_TOP_LEFT, out=out)

    ms = time_calls(torch, run, 20)
    tf = c.flops() / (ms * 1e-3) / 1e12
    res["prefill_qwen3_8b"] = dict(ms=round(ms, 4), tflops=round(tf, 1),
                                   frac=round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                                   seqlens=c.lens, flops=c.flops())
    ch = workloads.chunked_qwen3_8b("cuda")
    outc = torch.empty_like(ch.q)

    def runc(_):
        ops.prefill_paged(ch.q, ch.k_cache, ch.v_cache, ch.block_tables, ch.q_start, ch.q_len,
                          ch.context_lens, ch.chunk, out=outc)

    ms = time_calls(torch, runc, 20)
    tf = ch.flops() / (ms * 1e-3) / 1e12
    res["chunked_qwen3_8b"] = dict(ms=round(ms, 4), tflops=round(tf, 1),
                                   frac=round(tf / MFMA_BF16_PEAK_TFLOPS, 4), prior=ch.prior,
                                   chunk=ch.chunk, flops=ch.flops())
    for window in (False, True):
        v = workloads.vision_vl("cuda", window=window)
        cuv = v.cu_seqlens
        vs, vl = cuv[:-1].contiguous(), (cuv[1:] - cuv[:-1]).contiguous()
        outv = torch.empty_like(v.q)
        mv = max(v.lens)

        def runv(_):
            ops.prefill(v.q, v.k, v.v, vs, vl, vs, vl, mv, ops.CAUSAL_NONE, out=outv)

        # the windows' ~17 us launch is near the host's cost per call: timed back to back it
        # can measure the wrapper instead, so it is timed as 50 calls replayed from a graph
        ms = graph_call_ms(torch, runv) if window else time_calls(torch, runv, 30)
        tf = v.flops() / (ms * 1e-3) / 1e12
        # q, k, v read and the output written once: the windows (about 30 FLOP/B) sit
        # below the MFMA ridge, so their roofline is HBM bandwidth
        byts = 4 * v.q.numel() * v.q.element_size()
        if window:
            gbps = byts / (ms * 1e-3) / 1e9
            res[v.name + "_hbm"] = dict(gbps=round(gbps, 1), frac=round(gbps / HBM_PEAK_GBPS, 4),
                                        bytes=byts, bound="hbm",
                                        traffic=read_traffic("vision_window_qwen25vl",
                                                             PREFILL_SOURCES),
                                        timing="50 calls replayed from a HIP graph, median of 5")
        res[v.name] = dict(ms=round(ms, 4), tflops=round(tf, 1),
                           frac=round(tf / MFMA_BF16_PEAK_TFLOPS, 4), chunks=len(v.lens),
                           flops=v.flops())
    return res


def bench_kv_write_prefill(torch, ops, workloads):
    """KV write at prefill size: the causal prefill workload's K/V (all its tokens, 8 KV
    heads, D = 128) scattered into a paged cache through a shuffled slot mapping."""
    c = workloads.prefill_qwen3_8b("cuda")
    t, hk, d = c.k.shape
    bs = 16
    nblk = 2 * ((t + bs - 1) // bs)
    g = torch.Generator(device="cpu").manual_seed(7)
    blocks = torch.randperm(nblk, generator=g)[: (t + bs - 1) // bs]
    pos = torch.arange(t)
    slots = (blocks[pos // bs] * bs + pos % bs).to(torch.int64).cuda()
    kc = torch.zeros(nblk, hk, bs, d, dtype=c.k.dtype, device="cuda")
    vc = torch.zeros_like(kc)

    def run(_):
        ops.kv_write(c.k, c.v, kc, vc, slots)

    ms = time_calls(torch, run, 50)
    byts = 4 * t * hk * d * c.k.element_size() + 8 * t
    return dict(us=round(ms * 1e3, 2), tokens=t, bytes=byts,
                gbps=round(byts / (ms * 1e-3) / 1e9, 1),
                frac=round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                traffic=read_traffic("kv_write_prefill_qwen3_8b", KV_WRITE_SOURCES))


def bench_decode_vl(torch, ops, workloads):
    c = workloads.decode_vl("cuda", layers=DECODE_LAYERS)
    out = torch.empty_like(c.q)

    def decode(i):
        L = i % DECODE_LAYERS
        ops.paged_decode(c.q, c.k_cache[L], c.v_cache[L], c.block_tables, c.context_lens,
                         out=out)

    warm_up(torch, decode)
    ms = time_calls(torch, decode, 30)
    gbps = c.decode_bytes() / (ms * 1e-3) / 1e9
    return dict(ms=round(ms, 4), gbps=round(gbps, 1), frac=round(gbps / HBM_PEAK_GBPS, 4),
                bytes=c.decode_bytes(), traffic=read_traffic("decode_qwen25vl"),
                timing="median of 5 batches of 30 back-to-back calls")


def bench_decode_fp8(torch, ops, workloads, c):
    """Paged decode over the fp8 format of the same Qwen3-8B pool (e4m3 codes plus one
    fp32 scale per row, written by the fp8 KV-write kernel); GB/s of the fp8 bytes."""
    f8 = workloads.quantize_cache_fp8(c)
    out = torch.empty_like(c.q)

    def decode(i):
        L = i % DECODE_LAYERS
        ops.paged_decode(c.q, f8.k_cache[L], f8.v_cache[L], c.block_tables, c.context_lens,
                         out=out, k_scale=f8.k_scale[L], v_scale=f8.v_scale[L])

    warm_up(torch, decode)
    ms = time_calls(torch, decode, 30)
    byts = workloads.fp8_decode_bytes(c)
    gbps = byts / (ms * 1e-3) / 1e9
    del f8
    return dict(ms=round(ms, 4), gbps=round(gbps, 1), frac=round(gbps / HBM_PEAK_GBPS, 4),
                bytes=byts, traffic=read_traffic("decode_fp8_qwen3_8b"),
                format="e4m3 codes + fp32 scale per (token, KV head) row",
                timing="median of 5 batches of 30 back-to-back calls")


def bench_e2e(torch, mixed: bool, fp8_cache: bool = False):
    """Whole-model generation on the Qwen3-0.6B architecture (random-initialised bf16):
    64 prompts of U[128, 2048] random ids, 256 greedy tokens each.  ``mixed``:
    continuous batching with 1024-token prefill chunks and decodes packed into steps
    of up to 8192 tokens, the all-decode tail in a HIP graph; otherwise prefill-first
    (padded prefill batches of 8, then graph decode steps).  Throughput = (prompt +
    generated tokens) / elapsed."""
    from nano_inference_amd import e2e

    gen = e2e.build(use_graph=True, mixed=mixed, fp8_cache=fp8_cache)
    gen.run([pr[:64] for pr in gen.prompts[:4]])  # warm-up
    st = gen.run(gen.prompts)
    return dict(tokens_per_s=round(st.tokens_per_s, 1),
                decode_tokens_per_s=round(st.decode_tokens_per_s, 1),
                prompt_tokens=st.prompt_tokens, generated_tokens=st.generated_tokens,
                prefill_s=round(st.prefill_s, 4), decode_s=round(st.decode_s, 4),
                total_s=round(st.total_s, 4), steps=st.prefill_steps + st.decode_steps,
                scheduling="chunked prefill mixed with decodes" if mixed else "prefill first",
                kv_cache="fp8 (e4m3 + row scales)" if fp8_cache else "bf16")


def bench_e2e_eager(torch):
    """The Qwen3-0.6B generation of bench_e2e (prefill first) with every decode step run
    eagerly, layer by layer, as the reference engine runs it (no HIP graph), and the host
    time of every attention-path call: what the wrappers cost the CPU per call."""
    from nano_inference_amd import e2e

    gen = e2e.build(use_graph=False, mixed=False)
    gen.run([pr[:64] for pr in gen.prompts[:4]])  # warm-up
    with e2e.HostTimer() as ht:
        st = gen.run(gen.prompts)
    return dict(tokens_per_s=round(st.tokens_per_s, 1),
                decode_tokens_per_s=round(st.decode_tokens_per_s, 1),
                total_s=round(st.total_s, 4), scheduling="prefill first, eager decode steps",
                host_per_call=ht.per_call_us())


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_ms(fn, runs: int, budget_s: float) -> float:
    """One warm-up run, then the median of at least ``runs`` runs (more while the budget
    lasts, at most 50)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < runs or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2] * 1e3


def cpu_baseline(torch, workloads, budget_s: float = 20.0):
    """The reference's attention, op for op on the host cores (the oracle's restatement of
    layers/attention.py:12-50 and :267-332 and layers/vision.py:190-208), fp32, with the
    KV write loop and the attention timed apart: the small fp32 decode in full, and the
    Qwen3-8B decode, causal prefill and Qwen2.5-VL workloads on stated subsets (their padded fp32 scores would not
    fit or would take minutes).  One warm-up run, then the median of >= 5 runs.  The
    headline ``value`` is the decode subset's step (write + attention) in the units of
    the GPU line."""
    from oracle import reference_attention as ref
    from oracle import vision_windows as vw

    n = max(1, len(os.sched_getaffinity(0)))
    torch.set_num_threads(n)
    each = budget_s / 5

    def decode_leg(c, runs):
        kc, vc = c.k_cache[0], c.v_cache[0]
        mask = ref.decode_context_mask(c.context_lens)
        k4, v4 = c.k_new, c.v_new  # (B, 1, H_kv, D)
        slots = c.slot_mapping  # (B, 1)
        none = torch.full_like(slots, -1)  # attention alone: the loop finds no slot to write
        w_ms = _median_ms(lambda: ref.kv_write_loop(k4, v4, kc, vc, slots), runs, each / 4)
        a_ms = _median_ms(lambda: ref.paged_attention(c.q.unsqueeze(1), k4, v4, kc, vc, none,
                                                      c.block_tables, c.context_lens, mask,
                                                      is_prefill=False), runs, each)
        byts_a, byts_w = c.decode_bytes(), c.write_bytes()
        return dict(write_ms=round(w_ms, 3), attention_ms=round(a_ms, 3),
                    attention_gbps=round(byts_a / (a_ms * 1e-3) / 1e9, 3),
                    step_gbps=round((byts_a + byts_w) / ((a_ms + w_ms) * 1e-3) / 1e9, 3))

    legs = {}
    c1 = workloads.decode_small("cpu", torch.float32, 1001)
    legs["decode_small_full"] = dict(
        decode_leg(c1, 9), what="the small fp32 decode in full: batch 4, 16/8 heads, D 128, "
                                f"contexts {c1.lens}, block 16")
    lens2 = workloads.uniform_lengths(64, 512, 8192, 2002)[:8]
    pool = sum(math.ceil(L / 16) for L in lens2) + 64
    c2 = workloads.make_decode(8, 32, 8, 128, lens2, pool, 16, torch.float32, "cpu", 2002)
    legs["decode_qwen3_8b_subset"] = dict(
        decode_leg(c2, 5), what=f"the Qwen3-8B decode (batch 64), its first 8 sequences "
                                f"(contexts {lens2}), 32/8 heads, D 128")
    # causal prefill: the shortest of the 8 sequences, through the reference's prefill
    # branch (write loop over the step's tokens, repeat_interleave, causal sdpa)
    lens3 = workloads.uniform_lengths(8, 256, 4096, 3003)
    L3 = min(lens3)
    c3 = workloads.make_varlen([L3], 32, 8, 128, torch.float32, "cpu", 3003, True)
    q3, k3, v3 = (t.unsqueeze(0) for t in (c3.q, c3.k, c3.v))
    nb3 = math.ceil(L3 / 16) + 1
    kc3 = torch.zeros(nb3, 8, 16, 128)
    vc3 = torch.zeros_like(kc3)
    slots3 = torch.arange(L3, dtype=torch.int64).view(1, L3)
    none3 = torch.full_like(slots3, -1)
    w3 = _median_ms(lambda: ref.kv_write_loop(k3, v3, kc3, vc3, slots3), 5, each / 4)
    a3 = _median_ms(lambda: ref.paged_attention(q3, k3, v3, kc3, vc3, none3, None, None, None,
                                                is_prefill=True), 5, each)
    legs["prefill_qwen3_8b_subset"] = dict(
        write_ms=round(w3, 3), attention_ms=round(a3, 3),
        attention_gflops=round(c3.flops() / (a3 * 1e-3) / 1e9, 2),
        what=f"the Qwen3-8B causal prefill, its shortest sequence ({L3} tokens of {lens3}), "
             "32/8 heads")
    # vision: the first image (28 x 28 patches), full attention and its 64-token windows
    grid = [workloads.VISION_GRIDS[0]]
    cu_full = vw.full_cu_seqlens(grid)
    cu_win = vw.get_window_index(grid)[1]
    S5 = int(cu_full[-1])
    c5 = workloads.make_varlen([S5], 16, 16, 80, torch.float32, "cpu", 5105, False)
    fl_full = 4 * 16 * 80 * S5 * S5
    wl = [int(b - a) for a, b in zip(cu_win[:-1], cu_win[1:])]
    fl_win = 4 * 16 * 80 * sum(x * x for x in wl)
    af = _median_ms(lambda: ref.vision_attention(c5.q, c5.k, c5.v, cu_full), 5, each / 2)
    aw = _median_ms(lambda: ref.vision_attention(c5.q, c5.k, c5.v, cu_win), 5, each / 2)
    legs["vision_qwen25vl_subset"] = dict(
        full_ms=round(af, 3), full_gflops=round(fl_full / (af * 1e-3) / 1e9, 2),
        window_ms=round(aw, 3), window_gflops=round(fl_win / (aw * 1e-3) / 1e9, 2),
        what=f"the Qwen2.5-VL vision tower, its first image ({grid[0][1]}x{grid[0][2]} "
             f"patches, {S5} tokens), "
             f"16 heads, D 80: full attention and its {len(wl)} windows")
    lensv = workloads.uniform_lengths(32, 1024, 6144, 5005)[:4]
    poolv = sum(math.ceil(L / 16) for L in lensv) + 64
    cv = workloads.make_decode(4, 28, 4, 128, lensv, poolv, 16, torch.float32, "cpu", 5005)
    legs["decode_qwen25vl_subset"] = dict(
        decode_leg(cv, 5), what=f"the Qwen2.5-VL language decode (batch 32), its first 4 "
                                f"sequences (contexts {lensv}), 28/4 heads, D 128")
    head = legs["decode_qwen3_8b_subset"]
    return dict(value=head["step_gbps"], unit="GB/s", cores=torch.get_num_threads(),
                kind="port", cpu_model=_cpu_model(), threads=torch.get_num_threads(),
                sample=("reference decode step (per-token KV write loop + padded gather, "
                        "repeat_interleave, fp32 softmax) on the first 8 sequences of the "
                        "Qwen3-8B decode, fp32; "
                        "bytes counted at fp32 element size; the other legs as listed"),
                legs=legs)


PROFILE_WORKLOADS = ("decode", "decode_vl", "decode_fp8", "kv_write", "kv_write_prefill",
                     "prefill", "chunked", "vision_full", "vision_window")


def profile_run(torch, ops, workloads, name: str, n: int) -> None:
    """Minimal run for counter collection (rocprofv3 --pmc): three 1 GiB copies (the
    calibration of FETCH_SIZE / WRITE_SIZE against known bytes), then n launches of one
    workload's kernel(s) on the same inputs as the timed legs."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    del src, dst
    info = {}
    if name in ("decode", "decode_fp8", "kv_write"):
        c = workloads.decode_qwen3_8b("cuda", layers=DECODE_LAYERS)
        if name == "decode":
            for i in range(n):
                L = i % DECODE_LAYERS
                ops.paged_decode(c.q, c.k_cache[L], c.v_cache[L], c.block_tables, c.context_lens)
            info = dict(algorithmic_bytes=c.decode_bytes())
        elif name == "decode_fp8":
            f8 = workloads.quantize_cache_fp8(c)
            torch.cuda.synchronize()
            for i in range(n):
                L = i % DECODE_LAYERS
                ops.paged_decode(c.q, f8.k_cache[L], f8.v_cache[L], c.block_tables,
                                 c.context_lens, k_scale=f8.k_scale[L], v_scale=f8.v_scale[L])
            info = dict(algorithmic_bytes=workloads.fp8_decode_bytes(c))
        else:
            for i in range(n):
                L = i % DECODE_LAYERS
                ops.kv_write(c.k_new, c.v_new, c.k_cache[L], c.v_cache[L], c.slot_mapping)
            info = dict(algorithmic_bytes=c.write_bytes())
    elif name == "decode_vl":
        c = workloads.decode_vl("cuda", layers=DECODE_LAYERS)
        for i in range(n):
            L = i % DECODE_LAYERS
            ops.paged_decode(c.q, c.k_cache[L], c.v_cache[L], c.block_tables, c.context_lens)
        info = dict(algorithmic_bytes=c.decode_bytes())
    elif name == "kv_write_prefill":
        c = workloads.prefill_qwen3_8b("cuda")
        t, hk, d = c.k.shape
        bs = 16
        nblk = 2 * ((t + bs - 1) // bs)
        g = torch.Generator(device="cpu").manual_seed(7)
        blocks = torch.randperm(nblk, generator=g)[: (t + bs - 1) // bs]
        pos = torch.arange(t)
        slots = (blocks[pos // bs] * bs + pos % bs).to(torch.int64).cuda()
        kc = torch.zeros(nblk, hk, bs, d, dtype=c.k.dtype, device="cuda")
        vc = torch.zeros_like(kc)
        for _ in range(n):
            ops.kv_write(c.k, c.v, kc, vc, slots)
        info = dict(algorithmic_bytes=4 * t * hk * d * c.k.element_size() + 8 * t)
    elif name == "chunked":
        ch = workloads.chunked_qwen3_8b("cuda")
        outc = torch.empty_like(ch.q)
        for _ in range(n):
            ops.prefill_paged(ch.q, ch.k_cache, ch.v_cache, ch.block_tables, ch.q_start,
                              ch.q_len, ch.context_lens, ch.chunk, out=outc)
        info = dict(flops=ch.flops())
    elif name in ("prefill", "vision_full", "vision_window"):
        if name == "prefill":
            c = workloads.prefill_qwen3_8b("cuda")
            mode = ops.CAUSAL_TOP_LEFT
        else:
            c = workloads.vision_vl("cuda", window=name == "vision_window")
            mode = ops.CAUSAL_NONE
        cu = c.cu_seqlens
        qs, ql = cu[:-1].contiguous(), (cu[1:] - cu[:-1]).contiguous()
        out = torch.empty_like(c.q)
        for _ in range(n):
            ops.prefill(c.q, c.k, c.v, qs, ql, qs, ql, max(c.lens), mode, out=out)
        # q read and o written once, k and v read once
        info = dict(flops=c.flops(),
                    algorithmic_bytes=(2 * c.q.numel() + 2 * c.k.numel()) * c.q.element_size())
    else:
        raise SystemExit(f"bench.py: unknown profile workload {name!r}; one of "
                         f"{', '.join(PROFILE_WORKLOADS)}")
    torch.cuda.synchronize()
    print(json.dumps(dict(workload=name, launches=n, copy_bytes=1 << 30, **info)), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--profile", choices=PROFILE_WORKLOADS, default=None,
                    help="only run --launches launches of one workload (counter runs)")
    ap.add_argument("--launches", type=int, default=8)
    ap.add_argument("--no-e2e", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (--gpus {args.gpus} requested); "
              "the attention path has no multi-GPU leg", file=sys.stderr)
        return 2

    import torch

    from nano_inference_amd import ops, workloads

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    if args.profile:
        profile_run(torch, ops, workloads, args.profile, args.launches)
        return 0

    c, ms_step, dec_ms, dec_bracketed_ms, wr_ms = bench_decode(torch, ops, workloads, args.steps,
                                                               args.warmup)
    step_bytes = c.decode_bytes() + c.write_bytes()
    value = step_bytes / (ms_step * 1e-3) / 1e9
    dec_gbps = c.decode_bytes() / (dec_ms * 1e-3) / 1e9
    extra = {"decode_vl": bench_decode_vl(torch, ops, workloads)}
    extra["decode_qwen3_8b_fp8"] = bench_decode_fp8(torch, ops, workloads, c)
    extra.update(bench_prefill(torch, ops, workloads))
    pf = extra["prefill_qwen3_8b"]
    extra["kv_write_qwen3_8b"] = dict(us=round(wr_ms * 1e3, 2),
                                      gbps=round(c.write_bytes() / (wr_ms * 1e-3) / 1e9, 1),
                                      bytes=c.write_bytes(),
                                      traffic=read_traffic("kv_write_qwen3_8b", KV_WRITE_SOURCES))
    extra["kv_write_prefill_qwen3_8b"] = bench_kv_write_prefill(torch, ops, workloads)
    if not args.no_e2e:
        extra["e2e_qwen3_0p6b"] = bench_e2e(torch, mixed=True)
        extra["e2e_qwen3_0p6b_prefill_first"] = bench_e2e(torch, mixed=False)
        extra["e2e_qwen3_0p6b_fp8_cache"] = bench_e2e(torch, mixed=True, fp8_cache=True)
        extra["e2e_qwen3_0p6b_eager"] = bench_e2e_eager(torch)
    line = {
        "metric": "decode attn HBM GB/s (% of peak) + prefill attn TFLOP/s (% bf16 MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) q/k/v and KV pool, seeded",
        "config": {
            "workload": "paged decode, Qwen3-8B layout: B=64, 32/8 heads, D=128, "
                        "contexts U[512,8192], block 16, shuffled 40k-block pool; "
                        "step = KV write of 64 tokens + paged decode (one layer)",
            "batch": c.batch, "num_heads": c.num_heads, "num_kv_heads": c.num_kv_heads,
            "head_dim": c.head_dim, "block_size": 16, "pool_blocks": 40000,
            "context_tokens": sum(c.lens), "step_bytes": step_bytes,
        },
        "roofline": {
            "kernel": "paged decode (decode_split_kernel + decode_split_combine_kernel)",
            "bound": "hbm",
            "achieved": round(dec_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dec_gbps / HBM_PEAK_GBPS, 4),
            "traffic": read_traffic("decode_qwen3_8b"),
            "algorithmic_bytes": c.decode_bytes(),
            "us_per_launch": round(dec_ms * 1e3, 2),
            "timing": "back-to-back launches between two events, median of 5 rounds",
            "us_per_launch_own_events": round(dec_bracketed_ms * 1e3, 2),
        },
        "prefill": {
            "workload": "causal varlen prefill, Qwen3-8B layout, 8 seqs U[256,4096]",
            "tflops": pf["tflops"], "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": pf["frac"], "ms": pf["ms"],
        },
        "extra": extra,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(torch, workloads, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
