"""Benchmark of the MI355X attention hot path; prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-secondary] [--no-e2e]
                    [--only prefill|decode|ragged|paged|plumbing|copy|e2e]

A "step" is one call of the hot path on one batch of synthetic input, inputs resident in HBM:

  headline (value): causal prefill attention, 1 sequence x 12 q heads / 2 kv heads x 4096 tokens x
      head_dim 128, bf16 -> TFLOP/s (algorithmic flops 4*d*H*L(L+1)/2 over the measured time)
  secondary: paged decode, 64 rows with kv_len ~ U[128, 8192] in 16-token blocks under a permuted
      block table -> HBM GB/s (every visible K/V byte once + q, o, block table, lengths), with
      enough pool copies rotated per step that no step finds its K/V in the 256 MB MALL;
      ragged packed prefill, 16 sequences with L ~ U[16, 1024] -> TFLOP/s;
      paged prefill, the 4096-token causal prompt read through a permuted 16-token block table
      (the engine's prompt path) -> TFLOP/s;
      plumbing prefill, 1 x 12q/2kv x 512 causal fp32 (the reference's CPU-fallback case): the
      fp32 inputs on the GPU (the general kernel) -> TFLOP/s, beside their bf16 cast on the
      prefill kernel, the fp32 CPU fallback as its CPU baseline;
      end to end, the Qwen2.5-1.5B architecture (random bf16 weights) serving 16 concurrent chats
      (prompts U[32, 1000], 64 tokens each) through the scheduler -> generated tok/s.

Timing: each GPU workload first runs untimed for --ramp-ms (default 100 ms of wall time), which
brings the GPU from its idle clock state to the clock it sustains under the load (the 4096 prefill:
67-73 us per call over the first ~10 ms of calls from idle, a steady 60.0 us after 30 ms); then W
untimed warmup steps, then torch.cuda.synchronize(); a HIP event pair on the stream the kernels are
launched on brackets exactly K steps; synchronize.  The per-launch duration is the event time / K.
The headline also reports `cold_clock`: the same W + K steps timed right after the input upload,
before the ramp.  The CPU baseline is the fp32 SDPA oracle (the reference's fallback path) on the
same inputs, on this host's cores (median of 5-21 runs per workload).

--only runs one workload alone (for counter profiles: one kernel family per process); `copy` is a
1 GiB device-to-device copy of known size, the calibration for the FETCH_SIZE / WRITE_SIZE
counters.

One GPU only: --gpus N > 1 exits with a message.
"""
import argparse
import gc
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "my-inference-engine_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "prefill attn TFLOP/s + paged-decode attn HBM GB/s; e2e tok/s at 16 chats"
PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 dense bf16 flop/clk/CU
PEAK_HBM_GBS = 8000.0      # HBM3E
PEAK_FP32_TFLOPS = 157.3   # dense fp32 MFMA


RAMP_MS = 100.0  # set from --ramp-ms in main()


def _ramp(fn, ms):
    """Runs fn() untimed for at least `ms` milliseconds of wall time (batches of 10 calls, each
    batch synchronised), so that the GPU reaches the clock it sustains under this load: from idle
    the 1 x 12 x 4096 causal prefill takes 67-73 us per call for the first ~10 ms of calls and a
    steady 60.0 us after 30 ms or more."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        n += 10
    return n


def _time_gpu(fn, steps, warmup, ramp_ms=None):
    """(average ms per call of fn() over exactly `steps` calls, the shader clock they ran at):
    HIP events on the current stream, after the sustained-clock ramp (`_ramp`) and `warmup`
    untimed calls.  The timed calls run with the kernels' clock probe on (kernels.clock): the
    first work-group on each XCD of every attention launch counts its own shader cycles and
    real-time ticks, which give the clock the timed kernels ran at (None if no attention kernel
    ran).

    Python's garbage collector is run first and disabled from the ramp to the end of the timed
    calls (as timeit does): the host enqueues a call in 35-50 us against a 50-70 us kernel, so a
    collector pass of tens of milliseconds in the timed window -- the ramp's thousands of calls
    make one likely -- would leave the GPU idle inside it (seen: 0.7-1.05 ms per call instead of
    0.061), and one between the ramp and the timed calls would let the clock fall back."""
    import torch
    from kernels.clock import ClockProbe
    probe = ClockProbe()
    gc.collect()
    enabled = gc.isenabled()
    gc.disable()
    try:
        _ramp(fn, RAMP_MS if ramp_ms is None else ramp_ms)
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with probe:
            start.record()
            for i in range(steps):
                fn(i)
            end.record()
        torch.cuda.synchronize()
    finally:
        if enabled:
            gc.enable()
    return start.elapsed_time(end) / steps, probe.result()


def bench_prefill(steps, warmup, seq_len=4096, cold=False):
    """With cold=True also returns the time of the same steps right after the input upload, before
    the sustained-clock ramp (the GPU's idle clock state)."""
    import torch
    import workloads as wl
    from kernels.fa2 import FlashAttention2Function
    q, k, v = (t.cuda() for t in wl.prefill_single(seq_len, seed=0))
    fn = lambda i=0: FlashAttention2Function.apply(q, k, v, True, None)
    cold_ms = _time_gpu(fn, steps, warmup, ramp_ms=0.0)[0] if cold else None
    ms, clock = _time_gpu(fn, steps, warmup)
    flops = wl.causal_prefill_flops([seq_len])
    return (ms, flops, clock, cold_ms) if cold else (ms, flops, clock)


def bench_ragged(steps, warmup):
    import torch
    import workloads as wl
    from kernels.fa2 import fa2_varlen
    q, k, v, lens, cu = wl.prefill_ragged(seed=0)
    q, k, v = q.cuda(), k.cuda(), v.cuda()
    cu_t = torch.tensor(cu, dtype=torch.int32, device="cuda")
    mx = max(lens)
    ms, clock = _time_gpu(lambda i=0: fa2_varlen(q, k, v, cu_t, cu_t, mx, is_causal=True), steps,
                          warmup)
    return ms, wl.causal_prefill_flops(lens), lens, clock


def bench_paged_prefill(steps, warmup, seq_len=4096):
    """The prefill of a prompt whose K/V are already in the paged cache (the engine's path):
    1 x 12q/2kv x seq_len causal over 16-token blocks in a permuted order."""
    import torch
    import workloads as wl
    from kernels.fa2 import fa2_paged
    q, kp, vp, tables = wl.prefill_paged(seq_len, seed=0)
    q, kp, vp = q.cuda(), kp.cuda(), vp.cuda()
    bt = wl.table_tensor(tables).cuda()
    lens = torch.tensor([seq_len], dtype=torch.int32, device="cuda")
    ms, clock = _time_gpu(
        lambda i=0: fa2_paged(q, kp, vp, bt, lens, max_kv_len=seq_len, is_causal=True), steps, warmup)
    return ms, wl.causal_prefill_flops([seq_len]), clock


def bench_decode(steps, warmup, rotate_bytes=2 << 30):
    import torch
    import workloads as wl
    from kernels.fa2 import fa2_paged
    q, kp, vp, tables, lens = wl.decode_paged(seed=0)
    bt = wl.table_tensor(tables).cuda()
    lens_t = torch.tensor(lens, dtype=torch.int32, device="cuda")
    q = q.cuda()
    pool_bytes = 2 * kp.numel() * kp.element_size()
    copies = max(2, math.ceil(rotate_bytes / pool_bytes))
    pools = []
    for _ in range(copies):
        pools.append((kp.cuda(), vp.cuda()))
    max_kv = bt.shape[1] * 16

    def step(i=0):
        kpc, vpc = pools[i % copies]
        return fa2_paged(q, kpc, vpc, bt, lens_t, max_kv_len=max_kv)

    ms, clock = _time_gpu(step, steps, warmup)
    return ms, wl.decode_bytes(lens), lens, copies, clock


def bench_e2e(n_chats=16, reply_tokens=64, lo=32, hi=1000, seed=0, decode_graphs=True):
    """End-to-end serving of the Qwen2.5-1.5B architecture (28 layers, hidden 1536, 12q/2kv, head_dim
    128, SwiGLU 8960, vocab 151936, RoPE theta 1e6, tied embeddings) with random N(0, 0.02) bf16
    weights: n_chats conversations submitted at once, prompts of U[lo, hi] random token ids, each
    replying exactly reply_tokens tokens (no EOS) with seeded temperature-1 sampling, paged KV in
    16-token blocks under a 448 MiB budget (1024 blocks).  tok/s = generated tokens / wall time from
    the first submit to the last finish (metrics/benchmark_concurrency.py:57-76,166-172).

    The same chats run under both schedules: "mixed" packs admitted prompts into the decode step
    (every queued prompt that fits the step's token budget joins it), "separate" runs one prompt
    prefill per tick beside the decode step, as the reference's scheduler does (chat.py:247-253).
    With decode_graphs, steps without prompts replay HIP graphs captured once before the runs
    (batch buckets 1..n_chats); the capture time is reported, not counted, like a server's
    start-up.  Returns {"mixed": summary, "separate": summary} plus the workload's facts."""
    import torch
    from engine import Engine, run_concurrent_chats
    from kv_cache import KVCache
    from model import QWEN25_1P5B, Qwen2ForCausalLM
    cfg = QWEN25_1P5B
    with torch.device("cuda"):
        model = Qwen2ForCausalLM(cfg)
    model.init_random(std=0.02, seed=seed)
    model = model.to(torch.bfloat16).eval()
    cache = KVCache(1024, 16, "cuda", torch.bfloat16, cfg.num_layers, cfg.num_kv_heads, cfg.head_dim)
    kv_mib = cache.buf.numel() * cache.buf.element_size() / 2**20
    graphs, capture_s = None, 0.0
    if decode_graphs:
        from graphs import DecodeGraphs
        t0 = time.perf_counter()
        buckets = tuple(b for b in (1, 2, 4, 8, 16, 32, 64) if b < n_chats) + (n_chats,)
        graphs = DecodeGraphs(model, cache, buckets=buckets)
        torch.cuda.synchronize()
        capture_s = time.perf_counter() - t0
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n_chats,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lens]
    res = {"prompt_lens_sum": sum(lens), "kv_mib": kv_mib, "decode_graphs": bool(graphs),
           "graph_capture_s": capture_s}
    for name, mixed in (("separate", False), ("mixed", True)):
        eng = Engine(model, cache, max_reply_tokens=reply_tokens, temperature=1.0, seed=seed,
                     decode_graphs=graphs, mixed_prefill=mixed)
        run_concurrent_chats(eng, prompts[:2], reply_tokens=2)   # warm-up (two chats, two tokens)
        res[name] = run_concurrent_chats(eng, prompts, reply_tokens)
        assert cache.free_block_count() == cache.num_blocks
    # The reference's concurrency curve (metrics/benchmark_concurrency.py:17,204): the first n of
    # the same chats, mixed schedule, n = 1, 2, 4, 8 (n_chats is the run above).
    eng = Engine(model, cache, max_reply_tokens=reply_tokens, temperature=1.0, seed=seed,
                 decode_graphs=graphs, mixed_prefill=True)
    res["sweep"] = {n: run_concurrent_chats(eng, prompts[:n], reply_tokens)
                    for n in (1, 2, 4, 8) if n < n_chats}
    res["sweep"][n_chats] = res["mixed"]
    assert cache.free_block_count() == cache.num_blocks
    return res


def e2e_line(e2e):
    """The e2e secondary record: the mixed schedule's figures, the reference-style one beside."""
    m, s = e2e["mixed"], e2e["separate"]

    def figs(r):
        return {"tok_per_s": round(r["tok_per_s"], 1), "wall_s": round(r["wall_s"], 3),
                "ttft_p50_s": round(r["ttft_p50"], 4), "ttft_p99_s": round(r["ttft_p99"], 4),
                "lat_p50_s": round(r["lat_p50"], 4), "lat_p99_s": round(r["lat_p99"], 4),
                "tpot_s": round(r["tpot"], 5), "peak_active": r["peak_active"],
                "kv_util_pct": round(r["kv_util"], 1)}
    rec = {"metric": "e2e tok/s at 16 chats", "value": round(m["tok_per_s"], 1), "unit": "tok/s",
           "tokens": m["tokens"], "schedule": "mixed prefill+decode steps, decode-only steps "
           "replayed as HIP graphs, tokens drawn by the fused HIP sampler"}
    rec.update(figs(m))
    rec["separate_prefill"] = figs(s)
    rec["concurrency_sweep"] = [dict(chats=n, **figs(r)) for n, r in sorted(e2e["sweep"].items())]
    rec["workload"] = (f"Qwen2.5-1.5B architecture, random N(0,0.02) bf16 weights; 16 chats, "
                       f"prompts U[32,1000] random ids (sum {e2e['prompt_lens_sum']}), 64 tokens "
                       f"each, temperature 1, paged KV 1024 x 16-token blocks "
                       f"({e2e['kv_mib']:.0f} MiB)")
    rec["graph_capture_s"] = round(e2e["graph_capture_s"], 2)
    rec["cpu_baseline"] = None
    rec["cpu_baseline_note"] = ("not run: the 1.5B model over 16 x ~500-token prompts is hours of "
                                "CPU time, beyond the bench's minutes budget")
    return rec


def cpu_prefill_baseline(seq_len=4096, runs=5):
    import torch
    import workloads as wl
    from oracle import sdpa
    q, k, v = (t.float() for t in wl.prefill_single(seq_len, seed=0))
    sec = _median_time(lambda: sdpa.attention_ref(q, k, v, True), runs)
    return wl.causal_prefill_flops([seq_len]) / sec / 1e12, torch.get_num_threads(), sec


def _median_time(fn, runs):
    fn()  # warm up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_ragged_baseline(runs=7):
    """The reference's CPU path for a ragged batch: fp32 SDPA row by row, each row's causal mask
    aligned to its end (kernels/test_fa2.py:28-35, model.py:186-195), over the packed rows."""
    import torch
    import workloads as wl
    from oracle import sdpa
    q, k, v, lens, cu = wl.prefill_ragged(seed=0)
    q, k, v = q.float(), k.float(), v.float()
    sec = _median_time(lambda: sdpa.varlen_ref(q, k, v, cu, cu, True), runs)
    return wl.causal_prefill_flops(lens) / sec / 1e12, torch.get_num_threads(), sec


def bench_plumbing(steps, warmup, seq_len=512, cpu_runs=21, cpu=True):
    """The reference's plumbing case: 1 x 12q/2kv x 512 x 128 causal, fp32 N(0,1) seed 0.  Its
    own path is the CPU SDPA fallback (model.py:104-107, the is_causal branch of a fresh prefill),
    timed here on the host; the GPU runs the fp32 inputs themselves (the general kernel) and their
    bf16 cast (the prefill kernel) through FlashAttention2Function.apply."""
    import torch
    import workloads as wl
    from kernels.fa2 import FlashAttention2Function
    from model import sdpa_fallback
    q, k, v = wl.prefill_single(seq_len, dtype=torch.float32, seed=0)
    flops = wl.causal_prefill_flops([seq_len])
    qf, kf, vf = (t.cuda() for t in (q, k, v))
    ms, clock = _time_gpu(lambda i=0: FlashAttention2Function.apply(qf, kf, vf, True, None), steps,
                          warmup)
    qb, kb, vb = (t.bfloat16() for t in (qf, kf, vf))
    ms16, clock16 = _time_gpu(lambda i=0: FlashAttention2Function.apply(qb, kb, vb, True, None),
                              steps, warmup)
    out = {"gpu_ms": ms, "gpu_ms_bf16": ms16, "flops": flops, "clock": clock, "clock_bf16": clock16}
    if cpu:
        sec = _median_time(lambda: sdpa_fallback(q, k, v, [0], 6), cpu_runs)
        out.update(cpu_sec=sec, cpu_threads=torch.get_num_threads())
    return out


def cpu_decode_baseline(runs=5):
    """The reference's CPU decode path: dense gather of every row's blocks (kv_cache.py:117-121)
    then fp32 SDPA per row; a 16-row sample of the 64-row workload."""
    import torch
    import workloads as wl
    from oracle import paged as opaged
    from oracle import sdpa
    q, kp, vp, tables, lens = wl.decode_paged(seed=0)
    q, kp, vp = q[:16].float(), kp.float(), vp.float()
    tables, lens = tables[:16], lens[:16]
    S = max(lens)

    def run():
        kd = opaged.gather_dense(kp, tables, S, 16)
        vd = opaged.gather_dense(vp, tables, S, 16)
        return sdpa.attention_ref(q, kd, vd, False, lens)

    sec = _median_time(run, runs)
    return wl.decode_bytes(lens) / sec / 1e9, torch.get_num_threads(), sec


def bench_copy(steps, warmup, nbytes=1 << 30):
    """A plain 1 GiB device copy: reads and writes exactly nbytes per launch."""
    import torch
    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    ms, clock = _time_gpu(lambda i=0: dst.copy_(src), steps, warmup)
    return ms, nbytes, clock


def run_only(which, steps, warmup):
    """One workload alone, one JSON line with its time per launch."""
    if which == "e2e":
        print(json.dumps(e2e_line(bench_e2e())), flush=True)
        return
    if which == "prefill":
        ms, flops, clock = bench_prefill(steps, warmup)
        rate, unit = flops / (ms * 1e-3) / 1e12, "TFLOP/s"
    elif which == "decode":
        ms, nbytes, _, _, clock = bench_decode(steps, warmup)
        rate, unit = nbytes / (ms * 1e-3) / 1e9, "GB/s"
    elif which == "paged":
        ms, flops, clock = bench_paged_prefill(steps, warmup)
        rate, unit = flops / (ms * 1e-3) / 1e12, "TFLOP/s"
    elif which == "ragged":
        ms, flops, _, clock = bench_ragged(steps, warmup)
        rate, unit = flops / (ms * 1e-3) / 1e12, "TFLOP/s"
    elif which == "plumbing":
        pl = bench_plumbing(steps, warmup, cpu=False)
        ms, rate, unit = pl["gpu_ms"], pl["flops"] / (pl["gpu_ms"] * 1e-3) / 1e12, "TFLOP/s"
        clock = pl["clock"]
    else:
        ms, nbytes, clock = bench_copy(steps, warmup)
        rate, unit = 2 * nbytes / (ms * 1e-3) / 1e9, "GB/s"
    print(json.dumps({"only": which, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 5),
                      "value": round(rate, 2), "unit": unit, "clock": clock,
                      "step_cycles": _cycles(ms, clock)}), flush=True)


def _traffic_file():
    path = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return {}


def read_traffic(name):
    """HBM bytes per launch recorded by the rocprofv3 --pmc summaries under profiles/, if any.
    A static record of that profiling session (named by `traffic_session`), not a measurement of
    this run."""
    return _traffic_file().get(name)


def traffic_session():
    return _traffic_file().get("session")


def _cycles(ms, clock):
    """Shader cycles of one step at the clock the timed steps ran at."""
    return round(ms * 1e-3 * clock["ghz"] * 1e9) if clock else None


def _roofline(bound, achieved, peak, unit, clock, ms, traffic_key=None):
    r = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
         "frac": round(achieved / peak, 4)}
    if traffic_key is not None:
        r["traffic"] = read_traffic(traffic_key)
        r["traffic_session"] = traffic_session()
    r["clock_ghz"] = clock["ghz"] if clock else None
    r["clock_xcd_range_ghz"] = [clock["min"], clock["max"]] if clock else None
    r["step_cycles"] = _cycles(ms, clock)
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-secondary", action="store_true", help="prefill headline only")
    ap.add_argument("--no-e2e", action="store_true", help="skip the 16-chat end-to-end run")
    ap.add_argument("--only", choices=("prefill", "decode", "ragged", "paged", "plumbing", "copy",
                                       "e2e"),
                    help="run one workload alone (counter profiles)")
    ap.add_argument("--ramp-ms", type=float, default=100.0,
                    help="untimed run of each GPU workload before its warmup, so that the GPU "
                         "reaches its sustained clock (0: none)")
    args = ap.parse_args()
    global RAMP_MS
    RAMP_MS = args.ramp_ms
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the attention path runs on a single MI355X "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.only:
        run_only(args.only, args.steps, args.warmup)
        return

    ms, flops, clock, cold_ms = bench_prefill(args.steps, args.warmup, cold=True)
    tflops = flops / (ms * 1e-3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "causal prefill attention, 1 sequence x 12 q heads / 2 kv heads x "
                               "4096 tokens x head_dim 128, bf16, N(0,1) seed 0",
                   "flops_per_step": flops},
        "clock_ramp_ms": RAMP_MS,
        "cold_clock": {"ms_per_step": round(cold_ms, 5),
                       "value": round(flops / (cold_ms * 1e-3) / 1e12, 2),
                       "note": "the same warmup + steps timed right after the input upload, before "
                               "the untimed sustained-clock ramp that precedes every timed workload"},
        "roofline": _roofline("mfma", tflops, PEAK_BF16_TFLOPS, "TFLOP/s", clock, ms,
                              "fa2_prefill_kernel"),
    }
    if not args.no_cpu:
        cpu_tflops, cores, sec = cpu_prefill_baseline()
        out["cpu_baseline"] = {"value": round(cpu_tflops, 4), "unit": "TFLOP/s", "cores": cores,
                               "kind": "port",
                               "sample": f"the same 1x12x4096 causal prefill in fp32 through the "
                                         f"SDPA oracle, median of 5 runs ({sec:.3f} s each)",
                               "host_cpu_count": os.cpu_count()}
    if not args.no_secondary:
        dms, dbytes, lens, copies, dclock = bench_decode(args.steps, args.warmup)
        gbs = dbytes / (dms * 1e-3) / 1e9
        dec = {"metric": "paged-decode attn HBM GB/s", "value": round(gbs, 1), "unit": "GB/s",
               "ms_per_step": round(dms, 5), "bytes_per_step": dbytes,
               "workload": f"paged decode, 64 rows x 12q/2kv x head_dim 128, kv_len U[128,8192] "
                           f"(sum {sum(lens)}), 16-token blocks, permuted block table, bf16; "
                           f"{copies} pool copies rotated so no step hits the MALL",
               "roofline": _roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", dclock, dms,
                                     "fa2_decode_kernel")}
        if not args.no_cpu:
            cgbs, cores, sec = cpu_decode_baseline()
            dec["cpu_baseline"] = {"value": round(cgbs, 3), "unit": "GB/s", "cores": cores,
                                   "kind": "port",
                                   "sample": f"16 of the 64 rows (their bytes over their time): "
                                             f"dense gather (kv_cache.py:117-121) + fp32 SDPA, "
                                             f"median of 5 runs ({sec:.3f} s each)"}
        rms, rflops, rlens, rclock = bench_ragged(args.steps, args.warmup)
        rt = rflops / (rms * 1e-3) / 1e12
        rag = {"metric": "ragged varlen prefill attn TFLOP/s", "value": round(rt, 2),
               "unit": "TFLOP/s", "ms_per_step": round(rms, 5), "flops_per_step": rflops,
               "workload": f"16 packed causal sequences, L ~ U[16,1024] (sum {sum(rlens)}), "
                           f"12q/2kv, head_dim 128, bf16",
               "roofline": _roofline("mfma", rt, PEAK_BF16_TFLOPS, "TFLOP/s", rclock, rms,
                                     "fa2_prefill_kernel_varlen")}
        if not args.no_cpu:
            ct, cores, sec = cpu_ragged_baseline()
            rag["cpu_baseline"] = {"value": round(ct, 4), "unit": "TFLOP/s", "cores": cores,
                                   "kind": "port",
                                   "sample": f"the same 16 packed sequences in fp32, SDPA row by "
                                             f"row with each row's bottom-right mask, median of 7 "
                                             f"runs ({sec:.4f} s each)"}
        pms, pflops, pclock = bench_paged_prefill(args.steps, args.warmup)
        pt = pflops / (pms * 1e-3) / 1e12
        pag = {"metric": "paged prefill attn TFLOP/s", "value": round(pt, 2), "unit": "TFLOP/s",
               "ms_per_step": round(pms, 5), "flops_per_step": pflops,
               "workload": "causal prefill, 1 x 12q/2kv x 4096 x 128 bf16, K/V read from the paged "
                           "pool through a permuted table of 16-token blocks",
               "roofline": _roofline("mfma", pt, PEAK_BF16_TFLOPS, "TFLOP/s", pclock, pms,
                                     "fa2_prefill_kernel_paged")}
        pl = bench_plumbing(args.steps, args.warmup, cpu=not args.no_cpu)
        gt = pl["flops"] / (pl["gpu_ms"] * 1e-3) / 1e12
        gt16 = pl["flops"] / (pl["gpu_ms_bf16"] * 1e-3) / 1e12
        plb = {"metric": "plumbing prefill attn TFLOP/s (fp32 on the GPU)", "value": round(gt, 2),
               "unit": "TFLOP/s", "ms_per_step": round(pl["gpu_ms"], 5), "flops_per_step": pl["flops"],
               "dtype": "f32",
               "workload": "causal prefill 1 x 12q/2kv x 512 x 128, fp32 N(0,1) seed 0, through "
                           "FlashAttention2Function.apply in fp32 (the general kernel)",
               "roofline": _roofline("mfma", gt, PEAK_FP32_TFLOPS, "TFLOP/s", pl["clock"],
                                     pl["gpu_ms"]),
               "bf16_cast": {"value": round(gt16, 2), "unit": "TFLOP/s",
                             "ms_per_step": round(pl["gpu_ms_bf16"], 5),
                             "frac_of_bf16_peak": round(gt16 / PEAK_BF16_TFLOPS, 4),
                             "clock_ghz": pl["clock_bf16"]["ghz"] if pl["clock_bf16"] else None,
                             "step_cycles": _cycles(pl["gpu_ms_bf16"], pl["clock_bf16"])}}
        if "cpu_sec" in pl:
            plb["cpu_baseline"] = {
                "value": round(pl["flops"] / pl["cpu_sec"] / 1e12, 4), "unit": "TFLOP/s",
                "cores": pl["cpu_threads"], "kind": "port",
                "sample": f"the fp32 original through the model's CPU SDPA fallback (the "
                          f"reference's own path for this case), median of 21 runs "
                          f"({pl['cpu_sec'] * 1e3:.2f} ms each)"}
        out["secondary"] = [dec, rag, pag, plb]
        if not args.no_e2e:
            out["secondary"].append(e2e_line(bench_e2e()))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
