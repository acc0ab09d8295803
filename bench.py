#!/usr/bin/env python3
"""bench.py - throughput of the MI355X attention hot path against its roofline,
with the reference's CPU path timed beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload prefill|decode|delta|small|published|bandwidth|gdn|kda|dense|gemm|mla|mixer|indexer|all]

A step is one call of the hot path over one batch of synthetic, HBM-resident
input. The headline workload (config.workload) is configs[2] of BASELINE.json,
the Qwen3-8B-shaped causal GQA prefill at 8k (32 q / 8 kv heads, head_dim
128, QK-RMSNorm + RoPE theta 1e6, bf16 in, fp32 accumulate): `value` is its
whole-step TFLOP/s (norm/RoPE/append + flash attention) with the algorithmic
count 2*D*Hq*S*(S+1). `configs` carries all five configurations in the same
form (value, roofline of the dominant kernel, cpu_baseline, parity);
`published_shape` the reference's one published attention measurement (128
queries after 384 cached, docs/apple-gpu-plan.md:114-118); `bandwidth` a
device copy and the reference's own bandwidth test (a bf16 GEMV over 512 MiB
of weights, src/gpu-testing.cpp:298-351); `next_rows` the paths either side
of the hot path.

`roofline` is for the dominant kernel of the step: algorithmic flops (or
bytes) per launch over its average duration, from hipEvents the backend
records around every launch on the stream it runs on. `cpu_baseline` is the
reference's own kernels::attention / deltaStep (compiled from its headers into
oracle/_ref, "reference"), or the C restatement ("port") where that library
is absent, timed on the host's cores on a bounded sample of the same workload.
The CPU leg also checks the GPU's output of the timed step against the
reference (or the restatement) on the same inputs, outside the timed region:
`parity` gives max-abs, rel-L2 and the reference's own maxAbs/rms
(src/gpu-testing.cpp:85-95).

Every workload first runs its step untimed for CLOCK_RAMP_S seconds: the
GPU's clock rises over its first ~15 ms of sustained work and falls back
while the host runs a CPU baseline, so a few warm-up steps alone would time
the ramp. Then the W warm-up steps, then exactly K timed steps.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "math-utils_amd"))

PEAK_MFMA_F16 = 2516.6      # TFLOP/s, dense bf16/fp16 MFMA (MI355X spec)
PEAK_MFMA_F32 = 157.3       # TFLOP/s, fp32
PEAK_HBM = 8000.0           # GB/s
CPU_THREADS_CAP = 16        # the GPU box's CPU share for one GPU

# HBM bytes per launch of prefill_flash_kernel<128, 8, 2, 128, true> on
# rocprofv3 FETCH_SIZE and WRITE_SIZE passes (`--calibrate-copy
# --workload prefill`), each scaled by what the same counter reads for a
# 1 GiB device copy (fetch x2.000, write x1.000): 182.1 MB read + 136.3 MB
# written. Re-measure when the kernel changes.
PREFILL_FLASH_TRAFFIC = 318.4e6
# HBM bytes per launch of decode_attention_kernel<128> on configs[3], measured
# the same way (`--workload decode`): 1,240.4 MB read + 5.2 MB written
DECODE_ATTENTION_TRAFFIC = 1245.6e6
# HBM bytes per step of the two-level delta scan on configs[4] (pass A, the
# join and pass C together; `--workload delta`, the same scaling): pass A
# 340.0 MB read + 29.7 MB written, the join 27.3 + 12.6 MB, pass C 402.9 +
# 278.6 MB
DELTA_SCAN_TRAFFIC = 1091.1e6


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # the GPU's clock ramps over the first ~15 ms of sustained work: a short
    # warm-up times the ramp rather than the kernels
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="all",
                    choices=["prefill", "decode", "delta", "small", "published", "bandwidth", "gdn", "kda", "dense",
                             "gemm", "mla", "mixer", "indexer", "all"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="target CPU time of each baseline sample")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run a 1 GiB device copy first (scales HBM counters in profiles)")
    return ap.parse_args()


# ------------------------------------------------------------ synthetic data
class Xoshiro:
    """math::random::Random's randInt (Random.hpp:23-39, 67-86): only used to
    draw configs[3]'s sequence lengths exactly as the configuration states."""
    M = (1 << 64) - 1

    def __init__(self, seed):
        self.s = []
        x = seed
        for _ in range(4):
            x = (x + 0x9E3779B97F4A7C15) & self.M
            z = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & self.M
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & self.M
            self.s.append(z ^ (z >> 31))

    def next(self):
        s, M = self.s, self.M
        rotl = lambda v, k: ((v << k) | (v >> (64 - k))) & M  # noqa: E731
        r = (rotl((s[0] + s[3]) & M, 23) + s[0]) & M
        t = (s[1] << 17) & M
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
        return r

    def randint(self, lo, hi):
        span = hi - lo + 1
        limit = self.M - (self.M % span)
        while True:
            x = self.next()
            if x < limit:
                return lo + x % span


def rotary_table(dim, theta):
    import numpy as np
    j = np.arange(dim // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), np.float32(2) * j / np.float32(dim))).astype(np.float32)


def randn(shape, gen, dtype):
    import torch
    return torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32).to(dtype)


def gammas(dim, gen):
    import torch
    return (torch.rand((dim,), generator=gen, device="cuda") + 0.5).contiguous()


# ------------------------------------------------------------------ timing
CLOCK_RAMP_S = 0.25


def time_steps(step, steps, warmup, kernel, ramp_max=None):
    """clock ramp, W warm-up steps, then K timed steps between synchronisations;
    returns the step's ms, the named kernel's average launch ms from the
    backend's hipEvents, and all launched kernels' ms per step"""
    import torch
    import aigpu
    t = time.perf_counter()
    n = 0
    while time.perf_counter() - t < CLOCK_RAMP_S and (ramp_max is None or n < ramp_max):
        step()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # pass 1: the step as a caller runs it, no per-launch events
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    step_ms = t0.elapsed_time(t1) / steps
    # pass 2: the same steps with hipEvents around every launch
    aigpu.profile_reset()
    aigpu.profile(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    aigpu.profile(False)
    # a list of kernels: the sum of their average launch times (a scan of
    # several launches that run one after another)
    k_avg = 0.0
    for name in ([kernel] if isinstance(kernel, str) else kernel):
        k_ms, n = aigpu.profile_read(name)
        k_avg += k_ms / n if n else float("nan")
    all_ms, _ = aigpu.profile_read(None)
    return step_ms, k_avg, all_ms / steps


def parity(ref, got, max_abs_bar, rel_l2_bar=None, what=""):
    """max-abs and rel-L2 (the north star's bars) and the reference's own
    maxAbs/rms (src/gpu-testing.cpp:85-95) of got against ref"""
    import numpy as np
    ref = np.asarray(ref, np.float64).reshape(-1)
    got = np.asarray(got, np.float64).reshape(-1)
    diff = np.abs(ref - got)
    max_abs = float(diff.max()) if diff.size else 0.0
    norm = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(ref - got) / norm) if norm > 0 else max_abs
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    ok = bool(np.isfinite(got).all()) and max_abs <= max_abs_bar and (rel_l2_bar is None or rel <= rel_l2_bar)
    out = {"max_abs": max_abs, "rel_l2": rel, "ref_error": max_abs / rms if rms > 0 else max_abs,
           "bar": {"max_abs": max_abs_bar, "rel_l2": rel_l2_bar}, "pass": ok}
    if what:
        out["checked"] = what
    return out


def median_time(fn, runs=5, budget=None):
    """one warm-up, then the median of `runs` timings (fewer past `budget` s)"""
    fn()
    times = []
    t_all = time.perf_counter()
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
        if budget is not None and time.perf_counter() - t_all > budget:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_lib():
    """(library, kind): the reference's compiled kernels when present."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    ref = O.ref()
    threads = O.threads(0, cap=CPU_THREADS_CAP)
    if ref is not None:
        ref.ref_configure_pool(threads)
        return O, ref, "reference", threads
    return O, None, "port", threads


def cpu_model():
    """the host CPU's model string (/proc/cpuinfo), for the baseline record"""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_threads(cpu, n):
    """sizes the reference library's pool (or the port's thread count) to n"""
    O, ref, kind, threads = cpu
    if ref is not None:
        ref.ref_configure_pool(n)
    return n


# --------------------------------------------------------------- workloads
def prefill_workload(args, cpu):
    import numpy as np
    import torch
    import aigpu
    S, H, KV, D = 8192, 32, 8, 128
    gen = torch.Generator(device="cuda").manual_seed(2)
    q = randn((S, H, D), gen, torch.bfloat16)
    k = randn((S, KV, D), gen, torch.bfloat16)
    v = randn((S, KV, D), gen, torch.bfloat16)
    gq, gk = gammas(D, gen), gammas(D, gen)
    fr = torch.from_numpy(rotary_table(D, 1e6)).cuda()
    kc = torch.empty((KV, S, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    out = torch.empty((S, H, D), dtype=torch.float32, device="cuda")

    def step():
        aigpu.prefill(q, k, v, out, kc, vc, 0, H, KV, D, q_norm=gq, k_norm=gk, freqs=fr,
                      rotary_dims=D)

    flops = 2.0 * D * H * S * (S + 1)
    step_ms, k_ms, launched_ms = time_steps(step, args.steps, args.warmup, "prefill_flash_kernel")
    aigpu.check_range()   # no fp16 range error in any timed call
    res = {
        "workload": "configs[2] qwen3-8b causal GQA prefill S=8192 32q/8kv D=128 bf16, QK-norm+RoPE",
        # bf16 in; the flash MFMAs take fp16 operands (3 more mantissa bits) and accumulate in fp32
        "dtype": "fp16",
        "value": flops / (step_ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": step_ms,
        "kernels_ms_per_step": launched_ms,
        "roofline": {"kernel": "prefill_flash_kernel", "bound": "mfma",
                     "achieved": flops / (k_ms * 1e-3) / 1e12, "peak": PEAK_MFMA_F16,
                     "unit": "TFLOP/s", "frac": flops / (k_ms * 1e-3) / 1e12 / PEAK_MFMA_F16,
                     "traffic": PREFILL_FLASH_TRAFFIC, "kernel_ms": k_ms, "flops_per_launch": flops},
    }
    got = out.cpu().numpy()

    # the same prefill with a sliding window of 4096 keys (per-layer windows,
    # LocalModel.hpp:821-830; the first key a query sees, Kernels.hpp:142)
    W = 4096

    def step_window():
        aigpu.prefill(q, k, v, out, kc, vc, 0, H, KV, D, q_norm=gq, k_norm=gk, freqs=fr, rotary_dims=D, window=W)

    wflops = 4.0 * D * H * sum(min(i + 1, W) for i in range(S))
    w_step, w_k, _ = time_steps(step_window, args.steps, args.warmup, "prefill_flash_kernel")
    aigpu.check_range()
    res["window_4096"] = {"workload": "configs[2] shape with a sliding window of 4096 keys",
                          "value": wflops / (w_step * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": w_step,
                          "kernel_ms": w_k, "kernel_frac": wflops / (w_k * 1e-3) / 1e12 / PEAK_MFMA_F16,
                          "flops_per_launch": wflops}
    if cpu is not None:
        O, ref, kind, threads = cpu
        qh = q.float().cpu().numpy()
        kh = k.float().cpu().numpy()
        vh = v.float().cpu().numpy()
        # parity of the timed (full causal) step on 64 sampled query rows,
        # the last 16 (the longest histories) among them
        rows = sorted(set(range(0, S, S // 48)) | set(range(S - 16, S)))
        qn, kn = O.qk_norm_rope(qh, kh, S, 0, H, KV, D, D, gq.cpu().numpy(), gk.cpu().numpy(), 1e-6,
                                fr.cpu().numpy(), D)
        want = O.attention_strided(qn, kn, vh, S, 0, H, KV, D, D, KV * D, D, 0, rows=rows, nthreads=threads)
        res["parity"] = parity(want, got[rows], 2e-3, 1e-3,
                               f"{len(rows)} query rows x 32 heads (rows 0, 170, ..., and the last 16) "
                               f"against the C restatement of QK-norm, RoPE and kernels::attention")
        del qn, kn, want

        def run(n, nthreads):
            cpu_threads(cpu, nthreads)
            start = S - n
            qq = np.ascontiguousarray(np.resize(qh[-64:], (n, H, D)), np.float32)
            o = np.zeros(n * H * D, np.float32)
            t = time.perf_counter()
            if ref is not None:
                ref.ref_attention(qq.reshape(-1), kh.reshape(-1), vh.reshape(-1), o, n, start, H, KV, D,
                                  D, 0, 1)
            else:
                O.attention(qq, kh, vh, n, start, H, KV, D, D, nthreads=nthreads)
            dt = time.perf_counter() - t
            return 4.0 * D * H * sum(start + i + 1 for i in range(n)), dt

        f0, t0 = run(32, threads)
        n = int(min(S, max(32, 32 * args.cpu_seconds / max(t0, 1e-3))))
        f1, t1 = run(n, threads)
        # one core, on a third of the time
        g0, u0 = run(4, 1)
        n1 = int(min(S, max(4, 4 * args.cpu_seconds / 3 / max(u0, 1e-3))))
        g1, u1 = run(n1, 1)
        cpu_threads(cpu, threads)
        res["cpu_baseline"] = {"value": f1 / t1 / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": kind,
                               "cpu_model": cpu_model(),
                               "single_core": {"value": g1 / u1 / 1e12, "unit": "TFLOP/s",
                                               "sample": f"the last {n1} query rows on one thread "
                                                         f"({g1 / 1e9:.1f} GFLOP in {u1:.1f} s)"},
                               "sample": f"kernels::attention over the last {n} of the 8192 query rows "
                                         f"(full causal history, {f1 / 1e9:.1f} GFLOP in {t1:.1f} s, "
                                         f"fp32, static-split pool)"}
    return res


def decode_parity(O, q, k, v, kc, vc, lengths, gq, gk, fr, H, KV, D, threads):
    """the timed decode step's output against the C restatement: QK-norm and
    RoPE of each sequence's new q and k at its position, then
    kernels::attention over its cached positions [0, L) and the new token"""
    import numpy as np
    want = []
    for b, L in enumerate(lengths):
        qn, kn = O.qk_norm_rope(q[b].float().cpu().numpy().reshape(1, H, D),
                                k[b].float().cpu().numpy().reshape(1, KV, D), 1, L, H, KV, D, D,
                                gq, gk, 1e-6, fr, D)
        keys = np.concatenate([kc[b, :, :L].float().cpu().numpy().transpose(1, 0, 2), kn], 0)
        vals = np.concatenate([vc[b, :, :L].float().cpu().numpy().transpose(1, 0, 2),
                               v[b].float().cpu().numpy().reshape(1, KV, D)], 0)
        want.append(O.attention(qn, keys, vals, 1, L, H, KV, D, D, nthreads=threads)[0])
    return np.stack(want)


def decode_workload(args, cpu):
    import numpy as np
    import torch
    import aigpu
    B, H, KV, D = 32, 32, 4, 128
    r = Xoshiro(3)
    lengths = [r.randint(1024, 32768) for _ in range(B)]
    cap = max(lengths) + 1
    gen = torch.Generator(device="cuda").manual_seed(3)
    q = randn((B, H, D), gen, torch.bfloat16)
    k = randn((B, KV, D), gen, torch.bfloat16)
    v = randn((B, KV, D), gen, torch.bfloat16)
    gq, gk = gammas(D, gen), gammas(D, gen)
    fr = torch.from_numpy(rotary_table(D, 1e6)).cuda()
    kc = randn((B, KV, cap, D), gen, torch.bfloat16)
    vc = randn((B, KV, cap, D), gen, torch.bfloat16)
    pos = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    out = torch.empty((B, H, D), dtype=torch.float32, device="cuda")

    def step():
        aigpu.decode(q, k, v, out, kc, vc, pos, max(lengths), H, KV, D, q_norm=gq, k_norm=gk, freqs=fr,
                     rotary_dims=D)

    nbytes = 2048.0 * sum(L + 1 for L in lengths)
    step_ms, k_ms, launched_ms = time_steps(step, args.steps, args.warmup, "decode_attention_kernel")
    merge_ms, merge_n = aigpu.profile_read("decode_merge_kernel")   # pass 2 of time_steps
    res = {
        "workload": "configs[3] qwen3-30b-a3b batched ragged GQA decode B=32 L~U[1k,32k] 32q/4kv D=128 bf16 KV",
        "dtype": "bf16",
        "value": nbytes / (step_ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": step_ms,
        "step_frac": nbytes / (step_ms * 1e-3) / 1e9 / PEAK_HBM,
        "kernels_ms_per_step": launched_ms,
        "merge_kernel_ms": merge_ms / merge_n if merge_n else None,
        "kv_bytes": nbytes,
        "roofline": {"kernel": "decode_attention_kernel", "bound": "hbm",
                     "achieved": nbytes / (k_ms * 1e-3) / 1e9, "peak": PEAK_HBM, "unit": "GB/s",
                     "frac": nbytes / (k_ms * 1e-3) / 1e9 / PEAK_HBM, "traffic": DECODE_ATTENTION_TRAFFIC,
                     "kernel_ms": k_ms, "bytes_per_launch": nbytes},
    }
    if cpu is not None:
        O, ref, kind, threads = cpu
        got = out.cpu().numpy()
        want = decode_parity(O, q, k, v, kc, vc, lengths, gq.cpu().numpy(), gk.cpu().numpy(),
                             fr.cpu().numpy(), H, KV, D, threads)
        res["parity"] = parity(want, got, 2e-3, 1e-3, "all 32 sequences x 32 heads against the C restatement "
                                                      "of QK-norm, RoPE and kernels::attention")
        qh = q.float().cpu().numpy()

        def run(nthreads, budget):
            cpu_threads(cpu, nthreads)
            done_bytes, spent, seqs = 0.0, 0.0, 0
            for b in range(B):
                L = lengths[b]
                keys = np.ascontiguousarray(kc[b, :, :L + 1].float().cpu().numpy().transpose(1, 0, 2))
                vals = np.ascontiguousarray(vc[b, :, :L + 1].float().cpu().numpy().transpose(1, 0, 2))
                o = np.zeros(H * D, np.float32)
                t = time.perf_counter()
                if ref is not None:
                    ref.ref_attention(np.ascontiguousarray(qh[b]).reshape(-1), keys.reshape(-1),
                                      vals.reshape(-1), o, 1, L, H, KV, D, D, 0, 1)
                else:
                    O.attention(qh[b:b + 1], keys, vals, 1, L, H, KV, D, D, nthreads=nthreads)
                spent += time.perf_counter() - t
                done_bytes += 2048.0 * (L + 1)
                seqs += 1
                if spent > budget:
                    break
            return done_bytes / spent / 1e9, seqs

        value, seqs = run(threads, args.cpu_seconds)
        single, seqs1 = run(1, args.cpu_seconds / 3)
        cpu_threads(cpu, threads)
        res["cpu_baseline"] = {"value": value, "unit": "GB/s", "cores": threads, "kind": kind,
                               "cpu_model": cpu_model(),
                               "single_core": {"value": single, "unit": "GB/s",
                                               "sample": f"the first {seqs1} sequences on one thread"},
                               "sample": f"kernels::attention for {seqs} of the 32 sequences, one call each "
                                         f"(count=1, start=L_b) as the reference decodes, fp32 "
                                         f"position-major KV; GB/s on the same bf16 KV byte count"}
    del kc, vc

    # the same shape with every sequence at 32768 cached positions
    Lu = 32768
    kcu = randn((B, KV, Lu + 1, D), gen, torch.bfloat16)
    vcu = randn((B, KV, Lu + 1, D), gen, torch.bfloat16)
    posu = torch.full((B,), Lu, dtype=torch.int32, device="cuda")

    def step_uniform():
        aigpu.decode(q, k, v, out, kcu, vcu, posu, Lu, H, KV, D, q_norm=gq, k_norm=gk, freqs=fr, rotary_dims=D)

    ubytes = 2048.0 * B * (Lu + 1)
    u_step, u_k, u_all = time_steps(step_uniform, args.steps, args.warmup, "decode_attention_kernel")
    res["uniform_32k"] = {"workload": "B=32, every sequence at L=32768, 32q/4kv D=128 bf16 KV",
                          "value": ubytes / (u_step * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": u_step,
                          "step_frac": ubytes / (u_step * 1e-3) / 1e9 / PEAK_HBM,
                          "kernels_ms_per_step": u_all,
                          "kernel_ms": u_k, "kernel_frac": ubytes / (u_k * 1e-3) / 1e9 / PEAK_HBM,
                          "kv_bytes": ubytes}
    del kcu, vcu
    return res


def delta_workload(args, cpu):
    import numpy as np
    import torch
    import aigpu
    S, HK, HV, KD, VD = 16384, 16, 32, 128, 128
    gen = torch.Generator(device="cuda").manual_seed(4)
    q = randn((S, HK, KD), gen, torch.bfloat16)
    k = randn((S, HK, KD), gen, torch.bfloat16)
    v = randn((S, HV, VD), gen, torch.bfloat16)
    g = -torch.nn.functional.softplus(torch.randn((S, HV), generator=gen, device="cuda"))
    beta = torch.sigmoid(torch.randn((S, HV), generator=gen, device="cuda"))
    state = torch.zeros((HV, KD, VD), dtype=torch.float32, device="cuda")
    out = torch.empty((S, HV, VD), dtype=torch.float32, device="cuda")

    def step():
        state.zero_()
        aigpu.gated_delta_rule(q, k, v, state, out, g=g, beta=beta)

    # the step's algorithmic bytes: q, k, v (bf16), g and beta (fp32) in,
    # out (fp32) and the final state out
    nbytes = float(2 * S * HK * KD * 2 + S * HV * VD * 2 + 2 * S * HV * 4 + S * HV * VD * 4 + HV * KD * VD * 4)
    # the scan's own: q, k, v in, out and the state out, the state in (the
    # per-chunk records it reads are the solve's output, not the step's input)
    scan_bytes = float(2 * S * HK * KD * 2 + S * HV * VD * 2 + S * HV * VD * 4 + 2 * HV * KD * VD * 4)
    # the scan at this shape is the two-level scan: pass A, the join and pass
    # C run one after another
    scan_kernels = ["delta_seg_kernel<false>", "delta_join_kernel", "delta_seg_kernel<true>"]
    step_ms, k_ms, launched_ms = time_steps(step, args.steps, args.warmup, scan_kernels)
    flops = S * HV * (7.0 * KD * VD + 4.0 * VD)
    res = {
        "workload": "configs[4] qwen3-next gated delta rule S=16384 16qk/32v heads D=128 chunk 64 bf16 in, fp32 state",
        # products on bf16 MFMA, each fp32 operand split into a bf16 high and
        # low part (three products), accumulated and kept in fp32
        "dtype": "bf16x3",
        "value": nbytes / (step_ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": step_ms,
        "recurrence_tflops": flops / (step_ms * 1e-3) / 1e12,
        "roofline": {"kernel": " + ".join(scan_kernels), "bound": "hbm",
                     "achieved": scan_bytes / (k_ms * 1e-3) / 1e9, "peak": PEAK_HBM, "unit": "GB/s",
                     "frac": scan_bytes / (k_ms * 1e-3) / 1e9 / PEAK_HBM, "traffic": DELTA_SCAN_TRAFFIC,
                     "kernel_ms": k_ms, "bytes_per_launch": scan_bytes,
                     "all_kernels_ms": launched_ms, "all_kernels_frac": nbytes / (launched_ms * 1e-3) / 1e9 / PEAK_HBM,
                     "bytes_per_step": nbytes},
    }
    if cpu is not None:
        # the whole workload: the mixer's token loop around the reference's own
        # deltaStep (oracle/_ref), single-threaded as gatedDeltaNetMixer runs
        # it; the C restatement where the reference library is absent
        O, ref, kind, threads = cpu
        qh = q.float().cpu().numpy()
        kh = k.float().cpu().numpy()
        vh = v.float().cpu().numpy()
        gh = g.cpu().numpy()
        bh = beta.cpu().numpy()
        t = time.perf_counter()
        if ref is not None:
            want, want_state = O.ref_gated_delta_rule(qh, kh, vh, gh, bh)
            what = "the reference's kernels::deltaStep driven token by token (restated l2norm/q-scale glue)"
        else:
            want, want_state = O.gated_delta_rule(qh, kh, vh, gh, bh, nthreads=1)
            what = "the C restatement of deltaStep"
        dt = time.perf_counter() - t
        res["cpu_baseline"] = {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
                               "sample": f"all 16384 tokens x 32 value heads, single-threaded as "
                                         f"gatedDeltaNetMixer runs it ({dt:.1f} s): {what}"}
        # the timed step (state zeroed, then the whole sequence) against the
        # same run: every output row and the final state
        res["parity"] = parity(want, out.cpu().numpy(), 2e-3, 1e-3, f"all 16384 x 32 x 128 outputs against {what}")
        res["parity"]["state"] = parity(want_state, state.cpu().numpy(), 2e-3, 1e-3, "the final 32 x 128 x 128 state")
    return res


def kda_workload(args, cpu):
    """Kimi Delta Attention's recurrence at the Kimi-Linear shape (32 heads of
    128, keys and values the same width), the gates fused from the raw
    projections with the bounded (safe) form"""
    import torch
    import aigpu
    S, H, D = 16384, 32, 128
    gen = torch.Generator(device="cuda").manual_seed(6)
    q = randn((S, H, D), gen, torch.bfloat16)
    k = randn((S, H, D), gen, torch.bfloat16)
    v = randn((S, H, D), gen, torch.bfloat16)
    f = torch.randn((S, H, D), generator=gen, device="cuda")
    b = torch.randn((S, H), generator=gen, device="cuda")
    a_log = torch.randn((H,), generator=gen, device="cuda") * 0.5
    dt = torch.randn((H, D), generator=gen, device="cuda")
    state = torch.zeros((H, D, D), dtype=torch.float32, device="cuda")
    out = torch.empty((S, H, D), dtype=torch.float32, device="cuda")

    def step():
        state.zero_()
        aigpu.kda_rule(q, k, v, None, None, state, out, f=f, b=b, a_log=a_log, dt_bias=dt, safe_gate=True,
                       lower_bound=-5.0)

    # q, k, v bf16 + f fp32 + b + out fp32 + the state read and written + aLog, dtBias
    nbytes = float(3 * S * H * D * 2 + S * H * D * 4 + S * H * 4 + S * H * D * 4 + 2 * H * D * D * 4
                   + H * 4 + H * D * 4)
    step_ms, k_ms, launched_ms = time_steps(step, args.steps, args.warmup, "kda_scan_kernel")
    # fp32 MFMA work per (head, 64-token chunk) at D = 128: the solve's decayed
    # products (10 blocks x 2 x 16*16*128*2), P (20 x 16^3*2), W and Qt, Ut and
    # Ot (2 x 10 x 16*16*128*2 each); the scan's three 64x128x128 products
    chunks = S // 64
    scan_flop = 3 * 64 * D * D * 2.0 * chunks * H
    solve_flop = (10 * 2 * 16 * 16 * D * 2 + 20 * 16 ** 3 * 2 + 2 * 2 * 10 * 16 * 16 * D * 2) * float(chunks * H)
    res = {
        "workload": "kimi delta attention S=16384 32 heads D=128 chunk 64, raw gates (safe), bf16 in, fp32 state",
        "dtype": "f32",
        "value": nbytes / (step_ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": step_ms,
        "step_tflops": (scan_flop + solve_flop) / (step_ms * 1e-3) / 1e12,
        "roofline": {"kernel": "kda_scan_kernel", "bound": "mfma",
                     "achieved": scan_flop / (k_ms * 1e-3) / 1e12, "peak": PEAK_MFMA_F32, "unit": "TFLOP/s",
                     "frac": scan_flop / (k_ms * 1e-3) / 1e12 / PEAK_MFMA_F32, "traffic": None,
                     "kernel_ms": k_ms, "all_kernels_ms": launched_ms, "flop_per_launch": scan_flop,
                     "solve_flop": solve_flop, "bytes_per_step": nbytes},
    }
    if cpu is not None:
        # a bounded sample: the first n tokens of every head through the
        # reference's deltaStep with perKeyDecay, one thread (the reference
        # spreads heads over its pool; the sample's rate is per thread)
        O, ref, kind, threads = cpu
        n = S
        qh = q[:n].float().cpu().numpy()
        kh = k[:n].float().cpu().numpy()
        vh = v[:n].float().cpu().numpy()
        gh, bh = O.kda_gates(f[:n].cpu().numpy(), b[:n].cpu().numpy(), a_log.cpu().numpy(), dt.cpu().numpy(),
                             True, -5.0)
        t = time.perf_counter()
        if ref is not None:
            O.ref_kda_rule(qh, kh, vh, gh, bh)
            what = "the reference's kernels::deltaStep (perKeyDecay) driven token by token"
        else:
            O.kda_rule(qh, kh, vh, gh, bh, nthreads=1)
            what = "the C restatement of deltaStep (perKeyDecay)"
        dt_s = time.perf_counter() - t
        res["cpu_baseline"] = {"value": nbytes * (n / S) / dt_s / 1e9, "unit": "GB/s", "cores": 1, "kind": kind,
                               "sample": f"all {n} tokens x 32 heads, single-threaded "
                                         f"({dt_s:.1f} s): {what}"}
    return res


def dense_workload(args, cpu):
    """the resident decoder (aigpu_dense_*) on a Qwen3-0.6B-shaped model, bf16
    weights, one token per step at positions from 4096 on"""
    import numpy as np
    import torch
    import aigpu
    H, NL, NH, KV, D, I, V = 1024, 28, 16, 8, 128, 3072, 151936
    start = 4096
    ramp = 200   # clock-ramp steps at most; each step decodes the next position
    cap = start + ramp + args.warmup + 2 * args.steps + 8   # time_steps runs the steps twice
    gen = torch.Generator(device="cuda").manual_seed(7)

    def w(n, k):
        t = (torch.randn((n, k), generator=gen, device="cuda") / k ** 0.5).to(torch.bfloat16)
        keep.append(t)
        return {"ptr": t.data_ptr(), "kind": "bf16", "in": k, "out": n}

    keep = []
    rng = np.random.default_rng(7)
    layers = []
    for _ in range(NL):
        layers.append({"q": w(NH * D, H), "k": w(KV * D, H), "v": w(KV * D, H), "o": w(H, NH * D),
                       "gate": w(I, H), "up": w(I, H), "down": w(H, I),
                       "input_norm": rng.uniform(0.5, 1.5, H).astype(np.float32),
                       "post_norm": rng.uniform(0.5, 1.5, H).astype(np.float32),
                       "q_norm": rng.uniform(0.5, 1.5, D).astype(np.float32),
                       "k_norm": rng.uniform(0.5, 1.5, D).astype(np.float32), "window": 0})
    head = w(V, H)
    cache = rng.standard_normal((cap, KV * D)).astype(np.float32)
    cfg = dict(hidden=H, heads=NH, kv_heads=KV, head_dim=D, intermediate=I, vocab=V, capacity=cap,
               rotary_dims=D, eps=1e-6, theta=1e6)
    dec = aigpu.DenseDecoder(cfg, layers, head, rng.uniform(0.5, 1.5, H).astype(np.float32),
                             [cache] * NL, [cache] * NL, start)
    del cache
    emb = rng.standard_normal(H).astype(np.float32)
    state = {"pos": start}

    def step():
        dec.decode(emb, state["pos"])
        state["pos"] += 1

    step_ms, g_ms, launched_ms = time_steps(step, args.steps, args.warmup, "dense_gemv_kernel", ramp_max=ramp)
    gemv_total, gemv_n = aigpu.profile_read("dense_gemv_kernel")   # pass 2 of time_steps
    attn_total, attn_n = aigpu.profile_read("dense_attn_kernel")
    dec.close()
    del keep
    weight_bytes = 2.0 * (NL * (H * NH * D + 2 * H * KV * D + NH * D * H + 3 * H * I) + V * H)
    pos_mid = state["pos"] - args.steps * 0.5   # mean position of the profiled steps
    kv_bytes = NL * 2.0 * pos_mid * KV * D * 4
    gemv_ms = gemv_total / args.steps
    attn_ms = attn_total / args.steps
    return {
        "workload": "resident decoder, Qwen3-0.6B shape (28 layers, 16q/8kv x 128, 3072 MLP, 151936 vocab), "
                    "bf16 weights, fp32 cache, positions 4096+",
        "dtype": "f32", "value": 1e3 / step_ms, "unit": "tokens/s", "ms_per_step": step_ms,
        "kernels_ms_per_step": launched_ms, "bytes_per_step": weight_bytes + kv_bytes,
        "step_hbm_gbs": (weight_bytes + kv_bytes) / (step_ms * 1e-3) / 1e9,
        "attention_ms_per_step": attn_ms,
        "attention_gbs": kv_bytes / (attn_ms * 1e-3) / 1e9,
        "roofline": {"kernel": "dense_gemv_kernel (the step's projections, weight bytes over their summed time)",
                     "bound": "hbm", "achieved": weight_bytes / (gemv_ms * 1e-3) / 1e9, "peak": PEAK_HBM,
                     "unit": "GB/s", "frac": weight_bytes / (gemv_ms * 1e-3) / 1e9 / PEAK_HBM, "traffic": None,
                     "gemv_ms_per_step": gemv_ms, "launches_per_step": gemv_n / args.steps,
                     "weight_bytes": weight_bytes},
    }


def gemm_workload(args, cpu):
    """a prefill projection through aigpu_matmul_device: Qwen3-8B's q_proj
    shape, 8192 tokens x 4096 -> 4096, fp32 activations, bf16 weights"""
    import torch
    import aigpu
    M, K, N = 8192, 4096, 4096
    gen = torch.Generator(device="cuda").manual_seed(8)
    a = torch.randn((M, K), generator=gen, device="cuda")
    w = (torch.randn((N, K), generator=gen, device="cuda") / K ** 0.5).to(torch.bfloat16)
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    step_ms, k_ms, _ = time_steps(lambda: aigpu.matmul(a, w, out, "bf16"), args.steps, args.warmup, "gemm_dma_kernel")
    split_ms, split_n = aigpu.profile_read("split_a_kernel")   # pass 2 of time_steps
    flop = 2.0 * M * N * K
    return {
        "workload": "projection 8192 x 4096 -> 4096 (Qwen3-8B q_proj), fp32 a, bf16 w, fp32 out",
        "dtype": "bf16", "value": flop / (step_ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": step_ms,
        "split_a_ms": split_ms / split_n if split_n else None,
        "roofline": {"kernel": "gemm_dma_kernel", "bound": "mfma", "achieved": flop / (k_ms * 1e-3) / 1e12,
                     "peak": PEAK_MFMA_F16, "unit": "TFLOP/s", "frac": flop / (k_ms * 1e-3) / 1e12 / PEAK_MFMA_F16,
                     "traffic": None, "kernel_ms": k_ms,
                     "note": "two bf16 products per output (a split into high part and residual by "
                             "split_a_kernel before it), so the MFMA work is twice the algorithmic count"},
    }


def mixer_workload(args, cpu):
    """attentionMixer for a Qwen3-8B prefill of 8192 tokens through
    aigpu_prefill_mixer (the q projection, k and v as one GEMM with the
    norm/RoPE/append pass after it, flash attention, the o projection), and the same layer through the separate entry points
    (four matmuls, prefill attention with its own prep) for comparison"""
    import torch
    import aigpu
    S, HID, H, KV, D = 8192, 4096, 32, 8, 128
    gen = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn((S, HID), generator=gen, device="cuda")
    ws = {}
    for name, (n, k) in {"q": (H * D, HID), "k": (KV * D, HID), "v": (KV * D, HID), "o": (HID, H * D)}.items():
        w = (torch.randn((n, k), generator=gen, device="cuda") / k ** 0.5).to(torch.bfloat16)
        ws[name] = {"w": w, "kind": "bf16", "out": n, "in": k}
    gq, gk = gammas(D, gen), gammas(D, gen)
    fr = torch.from_numpy(rotary_table(D, 1e6)).cuda()
    kc = torch.zeros((KV, S, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    out = torch.empty((S, HID), dtype=torch.float32, device="cuda")

    def fused():
        aigpu.prefill_mixer(x, ws, out, kc, vc, 0, H, KV, D, q_norm=gq, k_norm=gk, freqs=fr, rotary_dims=D)

    qb = torch.empty((S, H, D), dtype=torch.float32, device="cuda")
    kb = torch.empty((S, KV, D), dtype=torch.float32, device="cuda")
    vb = torch.empty_like(kb)
    att = torch.empty((S, H, D), dtype=torch.float32, device="cuda")

    def separate():
        aigpu.matmul(x, ws["q"]["w"], qb.view(S, H * D), "bf16")
        aigpu.matmul(x, ws["k"]["w"], kb.view(S, KV * D), "bf16")
        aigpu.matmul(x, ws["v"]["w"], vb.view(S, KV * D), "bf16")
        aigpu.prefill(qb, kb, vb, att, kc, vc, 0, H, KV, D, q_norm=gq, k_norm=gk, freqs=fr, rotary_dims=D)
        aigpu.matmul(att.view(S, H * D), ws["o"]["w"], out, "bf16")

    sep_ms, _, _ = time_steps(separate, args.steps, args.warmup, "gemm_kernel")
    step_ms, gd_ms, _ = time_steps(fused, args.steps, args.warmup, "gemm_dma_kernel")
    aigpu.check_range()   # no fp16 range error in any timed call
    proj = 2.0 * S * HID * (2 * H * D + 2 * KV * D)
    attn = 2.0 * D * H * S * (S + 1)
    flop = proj + attn
    per_launch = proj / 3   # q, k | v together, o: three gemm_dma_kernel launches per step
    return {
        "workload": "attentionMixer prefill, Qwen3-8B layer (4096 hidden, 32q/8kv x 128), 8192 tokens, "
                    "fp32 x, bf16 weights, QK-norm + RoPE, bf16 cache",
        "dtype": "bf16", "value": S / (step_ms * 1e-3), "unit": "tokens/s", "ms_per_step": step_ms,
        "tflops": flop / (step_ms * 1e-3) / 1e12,
        "separate_entry_points_ms": sep_ms,
        "roofline": {"kernel": "gemm_dma_kernel (the q projection, k and v as one GEMM, the o projection)",
                     "bound": "mfma", "achieved": per_launch / (gd_ms * 1e-3) / 1e12, "peak": PEAK_MFMA_F16,
                     "unit": "TFLOP/s", "frac": per_launch / (gd_ms * 1e-3) / 1e12 / PEAK_MFMA_F16,
                     "traffic": None, "kernel_ms": gd_ms,
                     "note": "average launch over the three; the projections' algorithmic flops / 3 per launch; "
                             "fp32 activations are split into two bf16 products"},
    }


def indexer_workload(args, cpu):
    """selectKeys through aigpu_select_keys at DeepSeek-V3.2's indexer shapes
    in the pooled form (64 heads x 128, topK 2048, pools of 4; hidden 7168,
    q rank 1536, bf16 weights): a decode step against 32K positions, and a
    4096-token prefill from empty"""
    import torch
    import aigpu
    HID, QR, NI, DI, P, TOPK = 7168, 1536, 64, 128, 4, 2048
    CAP = 32768 + 8
    gen = torch.Generator(device="cuda").manual_seed(10)

    def wt(n, k):
        return {"w": (torch.randn((n, k), generator=gen, device="cuda") / k ** 0.5).to(torch.bfloat16),
                "kind": "bf16", "out": n, "in": k}

    ws = {"k": wt(DI, HID), "gate": wt(DI, HID), "q": wt(NI * DI, QR), "w": wt(NI, HID)}
    kn = torch.ones(DI, device="cuda")
    ape = torch.randn((P, DI), generator=gen, device="cuda")
    keys = torch.randn((CAP, DI), generator=gen, device="cuda")
    gates = torch.randn((CAP, DI), generator=gen, device="cuda")
    pools = torch.randn((CAP // P + 1, DI), generator=gen, device="cuda")
    i32 = dict(dtype=torch.int32, device="cuda")
    stride = TOPK // P * P + P

    def case(count, start):
        h = torch.randn((count, HID), generator=gen, device="cuda")
        qr = torch.randn((count, QR), generator=gen, device="cuda")
        ss, sn, sk = torch.empty(count, **i32), torch.empty(count, **i32), torch.empty(count * stride, **i32)
        return lambda: aigpu.select_keys(h, qr, ws, kn, None, ape, keys, gates, pools, ss, sn, sk, start, NI, DI,
                                         TOPK, P)

    dec_ms, score_ms, _ = time_steps(case(1, 32768), args.steps, args.warmup, "index_score_kernel")
    pre_ms, pre_score_ms, _ = time_steps(case(4096, 0), max(2, args.steps // 10), 2, "index_score_kernel")
    macs = (32769 // P) * NI * DI
    pre_macs = sum((t + 1) // P for t in range(4096) if (t + 1) // P > TOPK // P) * NI * DI
    return {
        "workload": "selectKeys, DeepSeek-V3.2 indexer shapes pooled by 4 (64 x 128 heads, topK 2048), bf16 weights: "
                    "decode step at 32K positions",
        "dtype": "f32", "value": 1e3 / dec_ms, "unit": "steps/s", "ms_per_step": dec_ms,
        "prefill_4096_ms": pre_ms,
        "roofline": {"kernel": "index_score_kernel", "bound": "valu",
                     "achieved": 2 * macs / (score_ms * 1e-3) / 1e12, "peak": 157.3, "unit": "TFLOP/s",
                     "frac": 2 * macs / (score_ms * 1e-3) / 1e12 / 157.3, "traffic": None, "kernel_ms": score_ms,
                     "prefill_kernel_ms": pre_score_ms,
                     "prefill_tflops": 2 * pre_macs / (pre_score_ms * 1e-3) / 1e12},
    }


def mla_workload(args, cpu):
    """multi-head latent attention decode: one token against 4096 cached
    latents, 128 heads, qk_nope 128, v 128, kv_lora_rank 512 (DeepSeek-V3 /
    GLM-5.3 attention shape), fp32 kv_b_proj"""
    import torch
    import aigpu
    H, DN, DV, C, L = 128, 128, 128, 512, 4096
    gen = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn((1, H, DN), generator=gen, device="cuda")
    lat = torch.randn((L + 1, C), generator=gen, device="cuda")
    kvb = torch.randn((H * (DN + DV), C), generator=gen, device="cuda") / C ** 0.5
    out = torch.empty((1, H, DV), dtype=torch.float32, device="cuda")
    scale = 1.0 / (DN + 64) ** 0.5
    step_ms, k_ms, launched_ms = time_steps(lambda: aigpu.latent_attention(q, lat, kvb, out, L, scale),
                                            args.steps, args.warmup, "latent_attn_kernel")
    nbytes = (L + 1) * C * 4.0 + kvb.numel() * 4.0
    return {
        "workload": "latent attention decode, 1 token at 4096, 128 heads, nope/v 128, rank 512, fp32",
        "dtype": "f32", "value": nbytes / (step_ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": step_ms,
        "roofline": {"kernel": "all four kernels (fold, attention, merge, unfold)", "bound": "hbm",
                     "achieved": nbytes / (launched_ms * 1e-3) / 1e9, "peak": PEAK_HBM, "unit": "GB/s",
                     "frac": nbytes / (launched_ms * 1e-3) / 1e9 / PEAK_HBM, "traffic": None,
                     "attn_kernel_ms": k_ms, "all_kernels_ms": launched_ms, "bytes_per_step": nbytes},
    }


def gdn_workload(args, cpu):
    """the steps either side of the recurrence at configs[4]'s shapes: the fused
    qkvz de-interleave + causal conv (K 4) + SiLU, then the gated norm"""
    import numpy as np
    import torch
    import aigpu
    S, HK, HV, KD, VD, K = 16384, 16, 32, 128, 128, 4
    G = HV // HK
    CW = 2 * HK * KD + HV * VD
    gen = torch.Generator(device="cuda").manual_seed(5)
    fused = randn((S, HK, 2 * KD + 2 * G * VD), gen, torch.bfloat16)
    ba = randn((S, HK, 2 * G), gen, torch.bfloat16)
    kernel = torch.randn((CW, K), generator=gen, device="cuda") * 0.5
    window = torch.zeros((K - 1, CW), dtype=torch.float32, device="cuda")
    q = torch.empty((S, HK, KD), dtype=torch.bfloat16, device="cuda")
    k = torch.empty_like(q)
    v = torch.empty((S, HV, VD), dtype=torch.bfloat16, device="cuda")
    z = torch.empty_like(v)
    a = torch.empty((S, HV), dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    core = randn((S, HV, VD), gen, torch.float32)
    gamma = torch.rand((VD,), generator=gen, device="cuda") + 0.5
    normed = torch.empty((S, HV, VD), dtype=torch.bfloat16, device="cuda")

    def step():
        aigpu.gdn_conv(fused, kernel, window, q, k, v, HK, HV, KD, VD, ba=ba, z=z, a=a, b=b)
        aigpu.gdn_gated_norm(core, z, gamma, normed)

    conv_bytes = (S * HK * (2 * KD + 2 * G * VD) * 2 + S * HK * 2 * G * 2 + CW * K * 4 + 2 * (K - 1) * CW * 4 +
                  S * CW * 2 + S * HV * VD * 2 + 2 * S * HV * 4)
    norm_bytes = S * HV * VD * (4 + 2 + 2) + VD * 4
    step_ms, k_ms, launched_ms = time_steps(step, args.steps, args.warmup, "gdn_conv_kernel")
    aigpu.profile_reset()
    aigpu.profile(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    aigpu.profile(False)
    n_ms, n = aigpu.profile_read("gdn_gated_norm_kernel")
    n_ms = n_ms / n if n else float("nan")
    res = {
        "workload": "configs[4] shapes: fused qkvz de-interleave + causal conv K=4 + SiLU (bf16 in/out), "
                    "gated RMSNorm x SiLU(z) (fp32 x, bf16 z/out); S=16384 16k/32v heads D=128",
        "dtype": "bf16", "unit": "GB/s", "ms_per_step": step_ms,
        "value": (conv_bytes + norm_bytes) / (step_ms * 1e-3) / 1e9,
        "roofline": {"kernel": "gdn_conv_kernel", "bound": "hbm",
                     "achieved": conv_bytes / (k_ms * 1e-3) / 1e9, "peak": PEAK_HBM, "unit": "GB/s",
                     "frac": conv_bytes / (k_ms * 1e-3) / 1e9 / PEAK_HBM, "traffic": None,
                     "kernel_ms": k_ms, "bytes_per_launch": float(conv_bytes)},
        "gated_norm": {"kernel": "gdn_gated_norm_kernel", "bound": "hbm", "kernel_ms": n_ms,
                       "achieved": norm_bytes / (n_ms * 1e-3) / 1e9, "peak": PEAK_HBM, "unit": "GB/s",
                       "frac": norm_bytes / (n_ms * 1e-3) / 1e9 / PEAK_HBM, "bytes_per_launch": float(norm_bytes)},
    }
    if cpu is not None:
        # the C restatement (the reference's header cannot be compiled here),
        # single-threaded as the mixer runs these loops, on the first 512 tokens
        O = cpu[0]
        n = 512
        fh = fused[:n].float().cpu().numpy()
        bh = ba[:n].float().cpu().numpy()
        kh = kernel.cpu().numpy()
        ch = core[:n].cpu().numpy()
        gh = gamma.cpu().numpy()
        t = time.perf_counter()
        qkv, zh, _, _ = O.gdn_deinterleave(fh, bh, HK, HV, KD, VD)
        O.gdn_conv(qkv, kh, np.zeros((K - 1, CW), np.float32))
        O.gdn_gated_norm(ch, zh, gh, 1e-6)
        dt = time.perf_counter() - t
        res["cpu_baseline"] = {"value": (conv_bytes + norm_bytes) * n / S / dt / 1e9, "unit": "GB/s", "cores": 1,
                               "kind": "port", "sample": f"the first {n} of 16384 tokens, fp32, single-threaded "
                                                         f"({dt:.2f} s): the C restatement"}
    return res


def cfg2_workload(args, cpu):
    """Qwen3-0.6B decode, one token against 4096 cached positions
    (latency-bound: 16.8 MB of K and V)"""
    import numpy as np
    import torch
    import aigpu
    H, KV, D, L = 16, 8, 128, 4096
    gen = torch.Generator(device="cuda").manual_seed(1)
    q = randn((1, H, D), gen, torch.bfloat16)
    k = randn((1, KV, D), gen, torch.bfloat16)
    v = randn((1, KV, D), gen, torch.bfloat16)
    kc = randn((1, KV, L + 1, D), gen, torch.bfloat16)
    vc = randn((1, KV, L + 1, D), gen, torch.bfloat16)
    gq, gk = gammas(D, gen), gammas(D, gen)
    fr = torch.from_numpy(rotary_table(D, 1e6)).cuda()
    pos = torch.tensor([L], dtype=torch.int32, device="cuda")
    o = torch.empty((1, H, D), dtype=torch.float32, device="cuda")

    def step():
        aigpu.decode(q, k, v, o, kc, vc, pos, L, H, KV, D, q_norm=gq, k_norm=gk, freqs=fr, rotary_dims=D)

    step_ms, k_ms, launched_ms = time_steps(step, max(args.steps, 50), args.warmup, "decode_attention_kernel")
    merge_ms, merge_n = aigpu.profile_read("decode_merge_kernel")
    nbytes = 2.0 * (L + 1) * KV * D * 2
    res = {"workload": "configs[1] qwen3-0.6b decode L=4096 16q/8kv D=128 bf16 KV, QK-norm+RoPE", "dtype": "bf16",
           "unit": "GB/s", "value": nbytes / (step_ms * 1e-3) / 1e9, "ms_per_step": step_ms,
           "kernels_ms_per_step": launched_ms, "merge_kernel_ms": merge_ms / merge_n if merge_n else None,
           "roofline": {"kernel": "decode_attention_kernel", "bound": "hbm",
                        "achieved": nbytes / (k_ms * 1e-3) / 1e9, "peak": PEAK_HBM, "unit": "GB/s",
                        "frac": nbytes / (k_ms * 1e-3) / 1e9 / PEAK_HBM, "traffic": None, "kernel_ms": k_ms,
                        "bytes_per_launch": nbytes,
                        "note": "latency-bound: 16.8 MB take 2.1 us at 8 TB/s"}}
    if cpu is not None:
        O, ref, kind, threads = cpu
        want = decode_parity(O, q, k, v, kc, vc, [L], gq.cpu().numpy(), gk.cpu().numpy(), fr.cpu().numpy(),
                             H, KV, D, threads)
        res["parity"] = parity(want, o.cpu().numpy(), 2e-3, 1e-3, "16 heads against the C restatement of QK-norm, "
                                                                  "RoPE and kernels::attention")
        qh = np.ascontiguousarray(q.float().cpu().numpy().reshape(-1))
        keys = np.ascontiguousarray(kc[0].float().cpu().numpy().transpose(1, 0, 2)).reshape(-1)
        vals = np.ascontiguousarray(vc[0].float().cpu().numpy().transpose(1, 0, 2)).reshape(-1)
        out = np.zeros(H * D, np.float32)

        def call(nthreads):
            cpu_threads(cpu, nthreads)
            if ref is not None:
                return lambda: ref.ref_attention(qh, keys, vals, out, 1, L, H, KV, D, D, 0, 1)
            return lambda: O.attention(qh.reshape(1, H, D), keys.reshape(-1, KV, D), vals.reshape(-1, KV, D), 1, L,
                                       H, KV, D, D, nthreads=nthreads)

        t1, n1 = median_time(call(1), 7)
        tp, npool = median_time(call(threads), 7)
        cpu_threads(cpu, threads)
        res["cpu_baseline"] = {"value": nbytes / tp / 1e9, "unit": "GB/s", "cores": threads, "kind": kind,
                               "cpu_model": cpu_model(), "ms": tp * 1e3,
                               "single_core": {"value": nbytes / t1 / 1e9, "unit": "GB/s", "ms": t1 * 1e3},
                               "sample": f"the whole call: kernels::attention (count=1, start=4096), fp32 "
                                         f"position-major KV, median of {npool} (pool) and {n1} (one thread) runs "
                                         f"after a warm-up; GB/s on the same bf16 KV byte count. The reference "
                                         f"threads attention only above 262144 work units (Kernels.hpp:165), so "
                                         f"this call runs on one thread either way"}
    return res


def cfg1_workload(args, cpu):
    """GPT-2-small MHA prefill, fp32, 128 tokens, through the
    fp32 drop-in aigpu_attention_device (position-major KV, as kernels::attention)"""
    import numpy as np
    import torch
    import aigpu
    S, H, D = 128, 12, 64
    gen = torch.Generator(device="cuda").manual_seed(0)
    qf = torch.randn((S, H, D), generator=gen, device="cuda")
    kf = torch.randn((S, H, D), generator=gen, device="cuda")
    vf = torch.randn((S, H, D), generator=gen, device="cuda")
    of = torch.empty((S, H, D), dtype=torch.float32, device="cuda")

    def step():
        aigpu.attention_device(qf, kf, vf, of, S, 0, H, H, D, D, H * D, D)

    step_ms, k_ms, launched_ms = time_steps(step, max(args.steps, 50), args.warmup, "attention_f32_tile_kernel")
    flops = 4.0 * D * H * S * (S + 1) / 2
    res = {"workload": "configs[0] gpt2-small MHA prefill fp32 S=128 12 heads D=64", "dtype": "f32",
           "unit": "TFLOP/s", "value": flops / (step_ms * 1e-3) / 1e12, "ms_per_step": step_ms,
           "roofline": {"kernel": "attention_f32_tile_kernel", "bound": "fp32",
                        "achieved": flops / (k_ms * 1e-3) / 1e12, "peak": PEAK_MFMA_F32, "unit": "TFLOP/s",
                        "frac": flops / (k_ms * 1e-3) / 1e12 / PEAK_MFMA_F32, "traffic": None, "kernel_ms": k_ms,
                        "flops_per_launch": flops, "kernels_ms_per_step": launched_ms,
                        "note": "latency-bound: 25.4 MFLOP take 0.16 us at the fp32 peak; the step is the "
                                "tiled kernel (keys split in two) and the merge of its records"}}
    if cpu is not None:
        O, ref, kind, threads = cpu
        qh, kh, vh = (np.ascontiguousarray(t.cpu().numpy()) for t in (qf, kf, vf))
        out = np.zeros(S * H * D, np.float32)

        def call(threaded):
            if ref is not None:
                return lambda: ref.ref_attention(qh.reshape(-1), kh.reshape(-1), vh.reshape(-1), out, S, 0, H, H, D,
                                                 D, 0, threaded)
            return lambda: O.attention(qh, kh, vh, S, 0, H, H, D, D, nthreads=threads if threaded else 1)

        cpu_threads(cpu, threads)
        call(0)()
        want = out.reshape(S, H, D).copy() if ref is not None else O.attention(qh, kh, vh, S, 0, H, H, D, D)
        res["parity"] = parity(want, of.cpu().numpy(), 1e-5, None,
                               "every output against the reference's own kernels::attention"
                               if ref is not None else "every output against the C restatement")
        t1, n1 = median_time(call(0), 7)
        tp, npool = median_time(call(1), 7)
        res["cpu_baseline"] = {"value": flops / tp / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": kind,
                               "cpu_model": cpu_model(), "ms": tp * 1e3,
                               "single_core": {"value": flops / t1 / 1e12, "unit": "TFLOP/s", "ms": t1 * 1e3},
                               "sample": f"the whole call: kernels::attention (count=128, start=0), threaded "
                                         f"(1536 query-head tasks of 64-key history: below the reference's "
                                         f"262144-unit threshold, Kernels.hpp:165, so one thread) and "
                                         f"serial; median of {npool} and {n1} runs after a warm-up"}
    return res


def published_workload(args, cpu):
    """the reference's one published attention measurement: 128 queries after
    384 cached tokens, 32 query / 8 kv heads, D = 128, 35.8 ms serial and
    3.2 ms parallel on an M5 Pro CPU (docs/apple-gpu-plan.md:114-118); here
    the same call on the GPU through the fp32 drop-in and through the bf16
    flash prefill, and the reference's own kernels::attention on the host"""
    import numpy as np
    import torch
    import aigpu
    n, start, H, KV, D = 128, 384, 32, 8, 128
    T = start + n
    gen = torch.Generator(device="cuda").manual_seed(12)
    q = torch.randn((n, H, D), generator=gen, device="cuda")
    keys = torch.randn((T, KV, D), generator=gen, device="cuda")   # position-major, as the reference
    vals = torch.randn((T, KV, D), generator=gen, device="cuda")
    out = torch.empty((n, H, D), dtype=torch.float32, device="cuda")
    flops = 4.0 * D * H * sum(start + i + 1 for i in range(n))

    def step_f32():
        aigpu.attention_device(q, keys, vals, out, n, start, H, KV, D, D, KV * D, D)

    f_ms, fk_ms, f_all = time_steps(step_f32, max(args.steps, 50), args.warmup, "attention_f32_tile_kernel")
    got_f32 = out.cpu().numpy()
    # the bf16 flash path: history in the head-major bf16 cache, the 128 new
    # rows through prep (no norm, no RoPE: kernels::attention alone)
    qb, kb, vb = q.to(torch.bfloat16), keys[start:].to(torch.bfloat16), vals[start:].to(torch.bfloat16)
    kc = torch.zeros((KV, T, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:, :start] = keys[:start].transpose(0, 1).to(torch.bfloat16)
    vc[:, :start] = vals[:start].transpose(0, 1).to(torch.bfloat16)
    out_b = torch.empty((n, H, D), dtype=torch.float32, device="cuda")

    def step_flash():
        aigpu.prefill(qb, kb, vb, out_b, kc, vc, start, H, KV, D)

    b_ms, bk_ms, b_all = time_steps(step_flash, max(args.steps, 50), args.warmup, "prefill_flash_kernel")
    aigpu.check_range()
    res = {"workload": "reference microbenchmark shape: 128 queries after 384 cached, 32q/8kv D=128 "
                       "(docs/apple-gpu-plan.md:114-118: 35.8 ms serial, 3.2 ms parallel on an M5 Pro CPU)",
           "flops": flops,
           "gpu_f32": {"entry": "aigpu_attention_device (fp32, position-major KV, kernels::attention semantics)",
                       "ms_per_step": f_ms, "kernel_ms": fk_ms, "kernels_ms_per_step": f_all,
                       "tflops": flops / (f_ms * 1e-3) / 1e12},
           "gpu_flash_bf16": {"entry": "aigpu_prefill_attention (bf16 in, fp16 MFMA; history conversion, prep, "
                                       "flash)", "ms_per_step": b_ms, "flash_kernel_ms": bk_ms,
                              "kernels_ms_per_step": b_all, "tflops": flops / (b_ms * 1e-3) / 1e12}}
    if cpu is not None:
        O, ref, kind, threads = cpu
        qh = np.ascontiguousarray(q.cpu().numpy())
        kh = np.ascontiguousarray(keys.cpu().numpy())
        vh = np.ascontiguousarray(vals.cpu().numpy())
        o = np.zeros(n * H * D, np.float32)

        def call(threaded):
            if ref is not None:
                return lambda: ref.ref_attention(qh.reshape(-1), kh.reshape(-1), vh.reshape(-1), o, n, start, H, KV,
                                                 D, D, 0, threaded)
            return lambda: O.attention(qh, kh, vh, n, start, H, KV, D, D, nthreads=threads if threaded else 1)

        cpu_threads(cpu, threads)
        call(0)()
        want = o.reshape(n, H, D).copy() if ref is not None else O.attention(qh, kh, vh, n, start, H, KV, D, D)
        res["gpu_f32"]["parity"] = parity(want, got_f32, 1e-5, None, "every output against kernels::attention")
        # the flash path's inputs are bf16: the reference sees the same
        # rounded values, widened
        qr, kr, vr = (np.ascontiguousarray(t.to(torch.bfloat16).float().cpu().numpy()) for t in (q, keys, vals))
        if ref is not None:
            ob = np.zeros(n * H * D, np.float32)
            ref.ref_attention(qr.reshape(-1), kr.reshape(-1), vr.reshape(-1), ob, n, start, H, KV, D, D, 0, 0)
            want_b = ob.reshape(n, H, D)
        else:
            want_b = O.attention(qr, kr, vr, n, start, H, KV, D, D)
        res["gpu_flash_bf16"]["parity"] = parity(want_b, out_b.cpu().numpy(), 2e-3, 1e-3,
                                                 "every output against kernels::attention on the same "
                                                 "bf16-rounded inputs, widened")
        t1, n1 = median_time(call(0), 5)
        tp, npool = median_time(call(1), 5)
        res["cpu_baseline"] = {"kind": kind, "cpu_model": cpu_model(), "cores": threads,
                               "serial_ms": t1 * 1e3, "parallel_ms": tp * 1e3,
                               "serial_tflops": flops / t1 / 1e12, "parallel_tflops": flops / tp / 1e12,
                               "sample": f"kernels::attention, serial and on the static-split pool of {threads} "
                                         f"threads, median of {n1} / {npool} runs after a warm-up"}
    return res


def bandwidth_workload(args, cpu):
    """what HBM delivers on this box, beside the 8 TB/s spec peak the HBM
    fractions use: a 1 GiB device-to-device copy, and the reference's own
    bandwidth test (src/gpu-testing.cpp:298-351): y = x W^T with W 65536 x
    4096 bf16 (512 MiB) and one row x, through aigpu_matmul_device's GEMV, and
    through the reference's matmulNTBF16 on the host"""
    import numpy as np
    import torch
    import aigpu
    a = torch.empty((1 << 28,), dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    c_ms, ck_ms, _ = time_steps(lambda: aigpu.copy_device(b, a), 20, 5, "copy_kernel")
    t_ms, _, _ = time_steps(lambda: b.copy_(a), 20, 5, "none")
    copy_bytes = 2.0 * a.numel() * 4
    del a, b
    K, N = 4096, 65536
    gen = torch.Generator(device="cuda").manual_seed(13)
    x = torch.randn((1, K), generator=gen, device="cuda")
    w = torch.randn((N, K), generator=gen, device="cuda").to(torch.bfloat16)
    y = torch.empty((1, N), dtype=torch.float32, device="cuda")
    g_ms, gk_ms, _ = time_steps(lambda: aigpu.matmul(x, w, y, "bf16"), max(args.steps, 20), args.warmup,
                                "gemv_kernel")
    wbytes = float(N * K * 2)
    res = {"workload": "HBM bandwidth: device copy and the reference's bf16 GEMV bandwidth test",
           "peak": PEAK_HBM, "unit": "GB/s",
           "device_copy": {"bytes": copy_bytes, "ms_per_step": c_ms, "kernel_ms": ck_ms,
                           "value": copy_bytes / (ck_ms * 1e-3) / 1e9,
                           "frac": copy_bytes / (ck_ms * 1e-3) / 1e9 / PEAK_HBM,
                           "what": "aigpu_copy_device (copy_kernel: 16-byte nontemporal loads and stores) of "
                                   "1 GiB, read + write bytes over the kernel's time"},
           "torch_copy": {"bytes": copy_bytes, "ms_per_step": t_ms, "value": copy_bytes / (t_ms * 1e-3) / 1e9,
                          "frac": copy_bytes / (t_ms * 1e-3) / 1e9 / PEAK_HBM,
                          "what": "torch copy_ of the same 1 GiB"},
           "gemv_bf16": {"bytes": wbytes, "ms_per_step": g_ms, "kernel_ms": gk_ms,
                         "value": wbytes / (gk_ms * 1e-3) / 1e9, "frac": wbytes / (gk_ms * 1e-3) / 1e9 / PEAK_HBM,
                         "what": "gemv_kernel, 512 MiB of bf16 weights against one fp32 row (weight bytes over "
                                 "kernel time, as the reference's test counts)"}}
    if cpu is not None:
        O, ref, kind, threads = cpu
        wh = w.view(torch.int16).cpu().numpy().view(np.uint16)
        xh = x.cpu().numpy()
        res["gemv_bf16"]["parity"] = parity(xh.astype(np.float64) @ O.unpack_bf16(wh).astype(np.float64).T,
                                            y.cpu().numpy(), 1e-3, 1e-5, "all 65536 outputs against an fp64 product")
        if ref is not None:
            out = np.zeros(N, np.float32)
            cpu_threads(cpu, threads)
            fn = lambda: ref.ref_matmul_nt_bf16(xh.reshape(-1), wh.ctypes.data, out, 1, K, N, 1)  # noqa: E731
            tp, runs = median_time(fn, 8)
            res["cpu_baseline"] = {"value": wbytes / tp / 1e9, "unit": "GB/s", "cores": threads, "kind": kind,
                                   "cpu_model": cpu_model(),
                                   "sample": f"the reference's matmulNTBF16 on the static-split pool, median of "
                                             f"{runs} runs after a warm-up"}
    return res


def calibrate_copy():
    """one 1 GiB device-to-device copy: the HBM counters of this known-size
    kernel scale the FETCH_SIZE/WRITE_SIZE readings of the attention kernels"""
    import torch
    a = torch.empty((1 << 28,), dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(each GPU box has one MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch  # noqa: F401
    import aigpu
    aigpu.require()
    if args.calibrate_copy:
        calibrate_copy()
    cpu = None if args.no_cpu else cpu_lib()
    want = args.workload
    run = lambda name: want in (name, "all")  # noqa: E731
    configs = {}
    if run("prefill"):
        configs["cfg3"] = prefill_workload(args, cpu)
    if run("decode"):
        configs["cfg4"] = decode_workload(args, cpu)
    if run("delta"):
        configs["cfg5"] = delta_workload(args, cpu)
    if run("small"):
        configs["cfg1"] = cfg1_workload(args, cpu)
        configs["cfg2"] = cfg2_workload(args, cpu)
    extra = {}
    if run("published"):
        extra["published_shape"] = published_workload(args, cpu)
    if run("bandwidth"):
        extra["bandwidth"] = bandwidth_workload(args, cpu)
    rows = {}
    for name, fn in (("gdn_neighbours", gdn_workload), ("kda_rule", kda_workload), ("resident_decoder", dense_workload),
                     ("projection_gemm", gemm_workload), ("latent_attention", mla_workload),
                     ("prefill_mixer", mixer_workload), ("indexer", indexer_workload)):
        key = {"gdn_neighbours": "gdn", "kda_rule": "kda", "resident_decoder": "dense", "projection_gemm": "gemm",
               "latent_attention": "mla", "prefill_mixer": "mixer", "indexer": "indexer"}[name]
        if run(key):
            rows[name] = fn(args, cpu)
    # the line's headline: configs[2] (prefill) when it ran, else the first that did
    order = ["cfg3", "cfg4", "cfg5", "cfg2", "cfg1"]
    head = next((configs[c] for c in order if c in configs), None)
    if head is None:
        head = next(iter(rows.values()), None) or next(iter(extra.values()))
    line = {
        "metric": "attn TFLOP/s (prefill) & KV GB/s (decode) as % roofline, 1 MI355X vs host CPU",
        "value": head.get("value"), "unit": head.get("unit"), "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head.get("ms_per_step"), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": head.get("dtype"),
        "data": "synthetic (torch seeded N(0,1) at each configuration's shape)",
        "config": {"workload": head.get("workload"), "device": aigpu.device_name()},
        "roofline": head.get("roofline"),
        "cpu_baseline": head.get("cpu_baseline"),
        "parity": head.get("parity"),
        "clock_ramp_s": CLOCK_RAMP_S,
    }
    details = {k: v for k, v in head.items() if k not in line and k != "workload"}
    if details:
        line["details"] = details
    line["configs"] = {c: configs[c] for c in ["cfg1", "cfg2", "cfg3", "cfg4", "cfg5"] if c in configs}
    line.update(extra)
    if rows:
        line["next_rows"] = rows
    print(json.dumps(line))


if __name__ == "__main__":
    main()
