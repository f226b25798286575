"""Benchmark of the MI355X sampler and fused selected-token log-prob (one GPU).

Default line (the driver's N=1 run): config E, the sort-heavy large-batch sampler
(4096 rows x vocab 151936 fp32, history 4096, T 0.6, repetition 1.05, top-k 1024,
top-p 0.98, min-p 0.05), a ``logprob`` object for config D (16384 tokens x hidden 7168 ->
vocab 129280 with the Token-TIS ratio, plus its backward), and an ``extra`` object with the
other configurations, each with its own roofline and CPU baseline: sampler B (256 x 151936
bf16, full-vocabulary draw), sampler A (8 x 129280 fp32, top-k 50 + top-p) and log-prob C
(8192 x 2048 -> 151936), plus the B=1 decode step of ``generate_group`` at V=151936.

A step is one launch over one batch with inputs already resident in HBM.  Times come
from HIP events on the stream the kernels are launched on, over K back-to-back steps.
The roofline ``achieved`` figure is algorithmic bytes (sampler) or FLOPs (log-prob)
per launch over the measured average launch time:
  sampler bytes/row = V*sizeof(logit) + L_hist*8 + 4 (u) + 8 (id) + 4 (lp) + 4 (kept)
  log-prob FLOPs/token = 2*H*V
``cpu_baseline`` times the C oracle (a port of the same specification) or the reference
expression on the host, on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "tiny-dsv41_amd"), str(ROOT)]

METRIC = "sampler rows/s @V=151936; fused logprob tok/s @H=7168; % of HBM/MFMA peak"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by
# the same counters on a plain 1 GiB copy (FETCH x 2.0, WRITE x 1.0); the commands and raw
# counts are in the profiles/ summaries of each kernel and workload.
MEASURED_TRAFFIC = {
    "sampler_E": 2_627_486_720 + 1_852_211,  # topk_kernel + select_kernel (profiles/sampler_topk_E.md)
    "sampler_B": 82_981_683 + 32_768,  # full_kernel (profiles/sampler_full_B.md)
    "sampler_E_full": 2_500_868_710 + 2_671_616,  # full_kernel (profiles/sampler_full_E_shape.md)
    "sampler_A": 4_951_450 + 318_464 + 79_872,  # sliced topk_kernel + merge_kernel (profiles/sampler_topk_A.md)
    "logprob_D": 46_112_195_686 + 1_048_576,
    "logprob_C": 7_592_285_070 + 1_245_184,  # fused_kernel + merge_kernel
    "logprob_grad_D": 45_297_095_573 + 4_384_320_091,
}


def sampler_bytes_per_row(vocab, esize, hist_len):
    return vocab * esize + hist_len * 8 + 4 + 8 + 4 + 4


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # A sampler step is about 0.5 ms: 100 timed steps after 20 warm-up steps measure the
    # steady state (20 steps after 5 read several percent slow on a fresh box).
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="E", choices=["A", "B", "E", "E_full", "E_topp", "E_topk50", "none"],
                    help="headline sampler config; E_full / E_topp / E_topk50: E's logits in another "
                         "mode (no penalties); 'none' runs only the log-prob leg (for profiling)")
    ap.add_argument("--logprob", default="D", choices=["C", "D", "none"])
    ap.add_argument("--logprob-steps", type=int, default=10)
    ap.add_argument("--no-backward", action="store_true", help="skip the log-prob backward timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other configurations and the decode step")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="time a plain device copy of this many bytes (PMC calibration) and exit")
    return ap.parse_args()


def events_time(fn, steps, warmup, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def copy_calibration(nbytes, steps, torch):
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    ms = events_time(lambda: dst.copy_(src), steps, 2, torch)
    print(json.dumps({"copy_bytes": nbytes, "ms": ms, "GBps": 2 * nbytes / ms / 1e6}), flush=True)


# Other modes on a configuration's logits: its temperature, no penalties, and these knobs.
#   full: the training default (rollout_manager/training.py:74-81), no truncation, so a
#         full-vocabulary inverse-CDF draw;
#   topp, topk50: serving mixes the reference forwards to vLLM (rollout_manager/backends/
#         vllm_actor.py:178-185): top-p 0.9 alone, top-k 50 alone.
SAMPLER_MODES = {
    "full": ({}, "training-default full-vocabulary inverse CDF"),
    "topp": ({"top_p": 0.9}, "top-p 0.9 alone, no penalties"),
    "topk50": ({"top_k": 50}, "top-k 50 alone, no penalties"),
}


def bench_sampler(name, steps, warmup, cpu_baseline, torch, cpu_seconds=10.0, mode=None):
    """One sampler configuration, or the configuration's logits in one of SAMPLER_MODES."""
    from dsv41_rocm import _lib, workloads

    dev = torch.device("cuda:0")
    print(f"[bench] generating sampler config {name} on the GPU", file=sys.stderr, flush=True)
    inp = workloads.sampler_inputs(name, device=dev)
    logits, history, uniforms, knobs = inp["logits"], inp["history"], inp["uniforms"], inp["knobs"]
    if mode:
        knobs = {"temperature": knobs.get("temperature", 1.0), **SAMPLER_MODES[mode][0]}
        history = history[:, :0]
        inp = dict(inp, history=history, knobs=knobs)
    rows, vocab = logits.shape
    ids = torch.empty(rows, dtype=torch.int64, device=dev)
    lps = torch.empty(rows, dtype=torch.float32, device=dev)
    kept = torch.empty(rows, dtype=torch.int32, device=dev)
    status = torch.empty(rows, dtype=torch.int32, device=dev)
    d = _lib.SamplerDesc()
    d.struct_size = ctypes.sizeof(_lib.SamplerDesc)
    d.rows, d.vocab = rows, vocab
    d.logits_dtype = _lib.DTYPE_F32 if logits.dtype == torch.float32 else _lib.DTYPE_BF16
    d.logits_row_stride = logits.stride(0)
    d.logits = logits.data_ptr()
    if history.shape[1]:
        d.history = history.data_ptr()
        d.history_row_stride = history.stride(0)
        d.hist_len = history.shape[1]
    d.uniforms = uniforms.data_ptr()
    d.temperature = knobs.get("temperature", 1.0)
    d.repetition_penalty = knobs.get("repetition_penalty", 1.0)
    d.presence_penalty = knobs.get("presence_penalty", 0.0)
    d.frequency_penalty = knobs.get("frequency_penalty", 0.0)
    d.top_k = knobs.get("top_k", 0)
    d.top_p = knobs.get("top_p", 1.0)
    d.min_p = knobs.get("min_p", 0.0)
    d.greedy = 0
    d.out_ids, d.out_logprob, d.out_kept, d.out_status = (ids.data_ptr(), lps.data_ptr(),
                                                          kept.data_ptr(), status.data_ptr())
    lib = _lib.load()
    ws_bytes = lib.dsv41_sampler_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step():
        _lib.check(lib.dsv41_sampler_run(ctypes.byref(d), ws.data_ptr(), ws_bytes, stream))

    ms = events_time(step, steps, warmup, torch)
    assert int(status.max().item()) == 0, "sampler reported a bad row"
    # The shader clock dips for the first few dozen launches of a fresh load (the GPU's
    # power management; E's time follows the clock), so a short run reads slower than the
    # same launches once the clock has settled.  Reported beside the contract's figure,
    # measured after it: it never enters `value`.
    steady_steps = 100
    steady_ms = events_time(step, steady_steps, 0, torch)
    esize = logits.element_size()
    per_row = sampler_bytes_per_row(vocab, esize, history.shape[1])
    achieved = per_row * rows / (ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": rows / (ms * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if esize == 4 else "bf16",
        "data": "synthetic",
        "config": {"workload": f"{name}: sampler {rows}x{vocab} "
                               f"{'fp32' if esize == 4 else 'bf16'}, history {history.shape[1]}"
                               + (f", {SAMPLER_MODES[mode][1]}" if mode else ""),
                   "rows": rows, "vocab": vocab, "hist_len": history.shape[1], **knobs},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": MEASURED_TRAFFIC.get(f"sampler_{name}" + (f"_{mode}" if mode else "")),
                     "bytes_per_row": per_row},
        "steady_state": {"steps": steady_steps, "ms_per_step": steady_ms,
                         "rows_per_s": rows / (steady_ms * 1e-3),
                         "hbm_frac": per_row * rows / (steady_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "note": "the next 100 steps after the timed ones, once the shader clock has "
                                 "settled; not part of value"},
    }
    if cpu_baseline:
        line["cpu_baseline"] = cpu_sampler_baseline(inp, knobs, torch, cpu_seconds)
    return line


def cpu_sampler_baseline(inp, knobs, torch, seconds=10.0):
    """C oracle (port of the same spec), one thread, on a bounded row sample of the batch;
    plus the reference's full-vocab expression (rollout.py:144-148) for context."""
    import numpy as np

    import oracle

    cores = len(os.sched_getaffinity(0))
    sample_rows = min(inp["logits"].shape[0], 512 if seconds >= 10.0 else 64)
    x = inp["logits"][:sample_rows].float().cpu().numpy()
    h = inp["history"][:sample_rows].cpu().numpy()
    u = inp["uniforms"][:sample_rows].cpu().numpy()
    t0 = time.perf_counter()
    n = 0
    while True:
        oracle.sample(x, uniforms=u, history=h, **knobs)
        n += sample_rows
        if time.perf_counter() - t0 > seconds:
            break
    dt = time.perf_counter() - t0
    out = {"value": n / dt, "unit": "rows/s", "cores": 1, "kind": "port",
           "sample": f"C oracle over the first {sample_rows} rows of the batch, repeated for "
                     f"{dt:.1f} s on 1 of {cores} host cores"}
    # reference expression, full-vocab (no penalties/truncation exist in the reference)
    xt = torch.from_numpy(x[:64])
    T = knobs.get("temperature", 1.0)
    g = torch.Generator().manual_seed(0)
    ref = {}
    for threads in (1, cores):
        torch.set_num_threads(threads)
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < min(3.0, seconds):
            for r in range(xt.shape[0]):
                lp = torch.log_softmax(xt[r] / T, dim=-1)
                p = lp.exp()
                tok = int(torch.multinomial(p, 1, generator=g).item())
                float(lp[tok])
            reps += xt.shape[0]
        ref[f"threads_{threads}"] = reps / (time.perf_counter() - t0)
    out["reference_expression_rows_per_s"] = ref
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: every GPU box here has one "
              "GPU, and the sampler's rows and the log-prob's tokens shard across GPUs with no exchange",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if args.copy_bytes:
        copy_calibration(args.copy_bytes, args.steps, torch)
        return
    cpu = not args.no_cpu_baseline
    if args.workload == "none":
        line = {}
    else:
        line = bench_sampler(args.workload.split("_")[0], args.steps, args.warmup, cpu, torch,
                             mode=args.workload.split("_", 1)[1] if "_" in args.workload else None)
        print(json.dumps({k: line[k] for k in ("value", "unit", "ms_per_step")}), file=sys.stderr, flush=True)
    if args.logprob != "none":
        line["logprob"] = bench_logprob(args.logprob, args.logprob_steps, 3, cpu, torch,
                                        backward=not args.no_backward)
    if not args.no_extra:
        extra = {}
        for name in ("B", "A"):
            if name != args.workload:
                extra[f"sampler_{name}"] = bench_sampler(name, 200, 20, cpu, torch, cpu_seconds=4.0)
                print(json.dumps({name: extra[f"sampler_{name}"]["ms_per_step"]}), file=sys.stderr, flush=True)
        extra["sampler_E_full"] = bench_sampler("E", 100, 20, cpu, torch, cpu_seconds=4.0, mode="full")
        print(json.dumps({"E_full": extra["sampler_E_full"]["ms_per_step"]}), file=sys.stderr, flush=True)
        if args.logprob != "C":
            extra["logprob_C"] = bench_logprob("C", 20, 3, cpu, torch, backward=False)
        extra["decode_B1"] = bench_decode(torch)
        line["extra"] = extra
    print(json.dumps(line), flush=True)


def bench_decode(torch, tokens=200, warmup=20):
    """The per-token sampling step of generate_group at batch 1 (rollout.py:144-148) on one
    [1, 151936] fp32 logits row resident on the GPU, wall clock per token:
    * reference: log_softmax(logits / T) on the GPU, the finite check (a sync), exp, the
      4V-byte copy to the host, torch.multinomial on one CPU thread (rl/config.py:45,
      pytorch_rl.py:39), and the behaviour log-prob read back (another sync);
    * race: sample_next(draw="exponential_race"), which draws the reference's token: V Exp(1)
      variates from the CPU generator (the reference's own RNG work), their 4V-byte copy to
      the GPU, the kernel, two scalars back;
    * inverse_cdf: sample_next(draw="inverse_cdf"): one uniform, the kernel, two scalars back."""
    from dsv41_rocm import sample_next, workloads

    dev = torch.device("cuda:0")
    row = workloads.sampler_inputs("B", rows=1, device=dev)["logits"].float()
    T = 1.0
    threads = torch.get_num_threads()
    torch.set_num_threads(1)

    def reference(g):
        log_probs = torch.log_softmax(row[0].float() / T, dim=-1)
        if not torch.isfinite(log_probs).all().item():
            raise ValueError("generation log probabilities contain non-finite values")
        probabilities = log_probs.exp().cpu()
        token = int(torch.multinomial(probabilities, 1, generator=g).item())
        return token, float(log_probs[token].item())

    def timed(fn):
        g = torch.Generator().manual_seed(1234)
        for _ in range(warmup):
            fn(g)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = [fn(g) for _ in range(tokens)]
        dt = (time.perf_counter() - t0) / tokens
        return dt * 1e6, out

    ref_us, ref_out = timed(reference)
    race_us, race_out = timed(lambda g: sample_next(row, T, generator=g, draw="exponential_race"))
    cdf_us, _ = timed(lambda g: sample_next(row, T, generator=g, draw="inverse_cdf"))
    # the race's host share: the V exponentials and their copy to the GPU
    V = row.shape[1]
    g = torch.Generator().manual_seed(1)
    t0 = time.perf_counter()
    for _ in range(tokens):
        e = torch.empty(1, V, dtype=torch.float32).exponential_(1, generator=g)
    fill_us = (time.perf_counter() - t0) / tokens * 1e6
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(tokens):
        e.to(dev)
    torch.cuda.synchronize()
    h2d_us = (time.perf_counter() - t0) / tokens * 1e6
    torch.set_num_threads(threads)
    same = sum(int(a[0] == b[0]) for a, b in zip(ref_out, race_out))
    return {
        "metric": "sampling step latency at batch 1 (rollout.py:144-148)",
        "unit": "us/token",
        "vocab": V,
        "tokens": tokens,
        "reference_step_us": ref_us,
        "race_us": race_us,
        "inverse_cdf_us": cdf_us,
        "race_host_exponentials_us": fill_us,
        "race_h2d_copy_us": h2d_us,
        "race_ids_equal_reference": f"{same}/{tokens}",
        "note": "wall clock per token, logits resident on the GPU, host on 1 thread as the reference sets it",
    }


def bench_logprob(name, steps, warmup, cpu_baseline, torch, backward=False):
    """Fused selected-token log-prob over one batch of config C or D (D adds the ratio)."""
    from dsv41_rocm import _lib, selected_log_probs, workloads

    cfg = workloads.LOGPROB_CONFIGS[name]
    dev = torch.device("cuda:0")
    print(f"[bench] generating log-prob config {name} on the GPU", file=sys.stderr, flush=True)
    inp = workloads.logprob_inputs(name, device=dev)
    x, w, t = inp["x"], inp["w"], inp["targets"]
    n, h = x.shape
    v = w.shape[0]
    behavior = None
    if cfg.ratio:
        lp0 = selected_log_probs(x, w, t, 1.0)[0]
        behavior = (lp0 + 0.05 * torch.randn(n, generator=inp["generator"], device=dev)).contiguous()
    lp = torch.empty(n, dtype=torch.float32, device=dev)
    ent = torch.empty(n, dtype=torch.float32, device=dev)
    ratio = torch.empty(n, dtype=torch.float32, device=dev)
    status = torch.empty(n, dtype=torch.int32, device=dev)
    d = _lib.LogprobDesc()
    d.struct_size = ctypes.sizeof(_lib.LogprobDesc)
    d.n_tokens, d.hidden, d.vocab = n, h, v
    d.x, d.x_row_stride, d.w, d.w_row_stride = x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0)
    d.targets = t.data_ptr()
    d.temperature = 1.0
    if behavior is not None:
        d.behavior, d.is_cap, d.out_ratio = behavior.data_ptr(), 2.0, ratio.data_ptr()
    d.out_logprob, d.out_entropy, d.out_status = lp.data_ptr(), ent.data_ptr(), status.data_ptr()
    lib = _lib.load()
    ws_bytes = lib.dsv41_logprob_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step():
        _lib.check(lib.dsv41_logprob_run(ctypes.byref(d), ws.data_ptr(), ws_bytes, stream))

    ms = events_time(step, steps, warmup, torch)
    assert int(status.max().item()) == 0, "log-prob reported a bad token"
    flops = 2.0 * n * h * v
    achieved = flops / (ms * 1e-3) / 1e12
    out = {
        "metric": "fused selected-token log-prob tok/s",
        "value": n / (ms * 1e-3),
        "unit": "tok/s",
        "ms_per_step": ms,
        "steps": steps,
        "dtype": "bf16",
        "config": {"workload": f"{name}: {n} tokens x hidden {h} -> vocab {v}"
                               + (", Token-TIS ratio" if cfg.ratio else ""),
                   "tokens": n, "hidden": h, "vocab": v},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / BF16_PEAK_TFLOPS, "traffic": MEASURED_TRAFFIC.get(f"logprob_{name}"),
                     "flops_per_token": 2.0 * h * v},
    }
    if backward:
        out["backward"] = bench_logprob_backward(x, w, t, lp, ent, steps, torch)
    if cpu_baseline:
        out["cpu_baseline"] = cpu_logprob_baseline(x, w, t, torch)
    return out


def bench_logprob_backward(x, w, t, lp, ent, steps, torch):
    """Backward of the fused log-prob for dL/dlogprob = 1 per token: the logit-gradient
    kernel (logits recomputed on MFMA, bf16 gradient written once) and the whole backward
    with the two GEMMs (hipBLASLt through torch) that produce dL/dx and dL/dw."""
    from dsv41_rocm import logprob as lpmod

    n, h = x.shape
    v = w.shape[0]
    hx, hw, ht = lpmod._prepare(x, w, t, 1.0)
    _, ent_, _, lse, _ = lpmod._forward(hx, hw, ht, 1.0, None, 2.0)
    glp = torch.ones(n, dtype=torch.float32, device=x.device)
    kern = events_time(lambda: lpmod.logits_grad(hx, hw, ht, 1.0, lse, ent_, glp, None), steps, 1, torch)
    full = events_time(lambda: lpmod.selected_log_probs_backward(hx, hw, ht, 1.0, lse, ent_, glp, None),
                       steps, 1, torch)
    flops = 2.0 * n * h * v
    name = "D" if (n, h, v) == (16384, 7168, 129280) else "C" if (n, h, v) == (8192, 2048, 151936) else "?"
    return {
        "ms_per_step": full,
        "value": n / (full * 1e-3),
        "unit": "tok/s",
        "flops_per_token": 3 * 2.0 * h * v,
        "tflops": 3 * flops / (full * 1e-3) / 1e12,
        "grad_kernel": {"ms": kern, "roofline": {"bound": "mfma", "achieved": flops / (kern * 1e-3) / 1e12,
                                                 "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                                 "frac": flops / (kern * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                                                 "flops_per_token": 2.0 * h * v,
                                                 "bf16_out_bytes": 2 * n * v,
                                                 "traffic": MEASURED_TRAFFIC.get(f"logprob_grad_{name}")}},
        "gemms": "dL/dx = G @ w and dL/dw = G^T @ x, torch.mm (hipBLASLt)",
    }


def cpu_logprob_baseline(x, w, t, torch):
    """The reference expression log_softmax(linear(x, w).float() / T).gather(targets)
    (model.py:682-683, native_lora.py:81-82) on the host, bf16 linear, on a token subset."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    wc = w.cpu()
    xc, tc = x.cpu(), t.cpu()

    def run(k):
        logits = torch.nn.functional.linear(xc[:k], wc).float() / 1.0
        return torch.log_softmax(logits, dim=-1).gather(-1, tc[:k, None]).squeeze(-1)

    t0 = time.perf_counter()
    run(16)
    per_tok = (time.perf_counter() - t0) / 16
    k = int(max(16, min(512, 15.0 / max(per_tok, 1e-6))))
    t0 = time.perf_counter()
    run(k)
    dt = time.perf_counter() - t0
    return {"value": k / dt, "unit": "tok/s", "cores": cores, "kind": "reference",
            "sample": f"reference expression (bf16 linear, fp32 log_softmax, gather) on the first {k} "
                      f"tokens, {dt:.1f} s on {cores} host cores"}


if __name__ == "__main__":
    main()
