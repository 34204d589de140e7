"""Benchmark: verified tok/s of speculative decoding on one MI355X.

Workload: Llama-3-8B-shape Q4_0 random-init model (32 layers,
d 4096, 32/8 heads, FFN 14336, vocab 128256, untied Q4_0 head), 512-token seeded uniform
prompt, greedy decoding with the seeded oracle drafter (k=4, alpha=0.8) over the
target's recorded greedy continuation.  A "step" is one speculative verify step: k+1
rows through the whole model on the GPU, per-row head + argmax, acceptance on the device.

value = tokens emitted by K timed steps / wall time of those K steps (prefill excluded,
weights and KV resident in HBM).  Also reported:
  config.full_decode : the whole 1024-token decode of the config (k in {2, 4, 8}, alpha in
                 {0.5, 0.8}), each a separate call after the timed steps;
  roofline     : the quantized GEMM family (all verify matmuls), algorithmic bytes per
                 launch over its average launch time measured with HIP events on the
                 session stream (a separate pass over the same workload);
  config.opt_in_split_attention : the same timed steps with the opt-in split-position attention
                 (nc_ctx_set_attention; not the reference's arithmetic, so not the headline) and
                 where its greedy stream first leaves the reference order's;
  cpu_baseline : the CPU oracle (C++ restatement of the reference's portable x86 path) on the
                 host's cores: verify steps of the same model at the workload's positions, on
                 min(16, nproc) threads and on the reference's default 4, plus a GPU-vs-CPU
                 greedy stream comparison on the same model.
Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA
# Host threads: the box's CPU share for one GPU is 16 cores, whatever nproc reports there.
HOST_THREADS = min(16, len(os.sched_getaffinity(0)))
REFERENCE_DEFAULT_THREADS = 4  # the reference's default worker count (src/main.rs:64, :549-551)
# rocprofv3 FETCH_SIZE + WRITE_SIZE summary of the verify GEMMs on this workload (each counter
# scaled by what it reads for a 256 MiB copy); the command that made it is in the file.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "verify_gemm_llama3-8b_q4_0_k4_pmc_traffic.md")
TRAFFIC_PROFILE_C4 = os.path.join(ROOT, "profiles", "config4_verify_gemm_llama3-70b_q4_0_pmc_traffic.md")


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


GEMM_KERNELS = {"auto": 0, "dot4": 1, "mfma": 2}  # NC_GEMM_KERNEL_*
GEMM_KERNEL = "auto"
ATTENTION_ORDERS = {"sequential": 0, "split": 1}  # NC_ATTN_*
ATTENTION = "sequential"
PASS_LAUNCHES = {"direct": 0, "graph": 1}  # NC_PASS_*
PASS_LAUNCH = "direct"


def make_ctx(nc):
    """Device context on GPU 0 with the --gemm-kernel dot-product path, the --attention
    summation order and the --pass-launch mode selected."""
    ctx = nc.Context(0)
    ctx.set_gemm_kernel(GEMM_KERNELS[GEMM_KERNEL])
    ctx.set_attention(ATTENTION_ORDERS[ATTENTION])
    ctx.set_pass_launch(PASS_LAUNCHES[PASS_LAUNCH])
    return ctx


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(img, cfg, args, tok_per_step, gpu_stream, stream_prompt):
    """The oracle on the host, on the same model.  (1) Verify-step time at the workload's
    positions: the session's KV rows 0..n_prompt are filled (a timing aid: a 512-token CPU
    prefill alone would take minutes), then k+1-row verify passes run at positions n_prompt..;
    tok/s = the GPU run's tokens per step (same seed, same drafter, same greedy stream) over the
    CPU's seconds per step.  Timed on HOST_THREADS threads and on the reference's default 4.
    (2) Greedy stream identity: the oracle's greedy continuation of a 16-token prompt against
    the GPU's, with the oracle's top-2 logit margin at the first divergence."""
    import numpy as np

    from oracle import oracle as O
    t0 = time.time()
    om = O.Model(data=img.tobytes(), nthreads=HOST_THREADS)
    log(f"oracle model loaded in {time.time() - t0:.1f}s")
    # (2) stream identity
    s = O.Session(om, 64, 16)
    preds, margins, _ = s.verify_greedy(stream_prompt, 0)
    cpu_stream, cpu_margins = [int(preds[-1])], [float(margins[-1])]
    for i in range(len(gpu_stream) - 1):
        p, m, _ = s.verify_greedy(np.array([cpu_stream[-1]], np.uint32), len(stream_prompt) + i)
        cpu_stream.append(int(p[0]))
        cpu_margins.append(float(m[0]))
    s.close()
    diverge = next((i for i, (a, b) in enumerate(zip(cpu_stream, gpu_stream)) if a != int(b)), None)
    identity = {"prompt_tokens": len(stream_prompt), "tokens": len(cpu_stream),
                "identical": diverge is None, "first_divergence": diverge,
                "cpu_top2_margin_at_divergence": None if diverge is None else cpu_margins[diverge],
                "min_cpu_top2_margin": round(min(cpu_margins), 6)}
    log(f"gpu vs cpu greedy stream: {identity}")
    # (1) verify-step time at positions n_prompt..
    batch = np.asarray(gpu_stream[:args.k + 1], np.uint32)
    timed = {}
    for th, steps in ((HOST_THREADS, args.cpu_steps), (REFERENCE_DEFAULT_THREADS, max(1, args.cpu_steps // 3))):
        om.set_threads(th)
        s = O.Session(om, args.n_prompt + args.k + 8, 16)
        s.fill_kv(args.n_prompt, 7)
        t1 = time.time()
        for i in range(steps):
            s.verify_greedy(batch, args.n_prompt + i)
        dt = (time.time() - t1) / steps
        s.close()
        timed[th] = (dt, steps)
        log(f"cpu verify step ({args.k + 1} rows at position {args.n_prompt}) on {th} threads: {dt:.2f} s")
    om.close()
    dt, steps = timed[HOST_THREADS]
    dt4, steps4 = timed[REFERENCE_DEFAULT_THREADS]
    return {"value": round(tok_per_step / dt, 4), "unit": "tok/s", "cores": HOST_THREADS, "kind": "port",
            "cpu_model": cpu_model_name(), "nproc": os.cpu_count(),
            "value_reference_default_threads": round(tok_per_step / dt4, 4),
            "reference_default_threads": REFERENCE_DEFAULT_THREADS,
            "seconds_per_verify_step": round(dt, 3), "seconds_per_verify_step_4_threads": round(dt4, 3),
            "sample": (f"same {args.config}-shape model on the host: {steps} verify passes of {args.k + 1} rows at "
                       f"positions {args.n_prompt}.. on {HOST_THREADS} threads ({steps4} on "
                       f"{REFERENCE_DEFAULT_THREADS}), KV rows 0..{args.n_prompt} filled; scaled by the GPU run's "
                       f"{tok_per_step:.3f} tokens per step"),
            "stream_vs_gpu": identity}


def _traffic_from(path):
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def measured_traffic(args):
    """HBM bytes per verify-GEMM launch from the committed counter summary, or None when
    the summary is absent or was taken on another workload."""
    if args.config != "llama-3-8b" or args.k != 4:
        return None
    return _traffic_from(TRAFFIC_PROFILE)


def _q4_0_random_blocks(M, K, seed):
    """Random valid Q4_0 blocks (uniform nibbles, f16 scales ~ N(0,0.02)/8): the GEMM's
    bandwidth does not depend on the values."""
    import numpy as np
    rng = np.random.default_rng(seed)
    blk = rng.integers(0, 256, (M, K // 32, 18), dtype=np.uint8)
    sc = (np.abs(rng.normal(0, 0.0025, (M, K // 32))) + 1e-4).astype(np.float16).view(np.uint16)
    blk[:, :, 0] = sc & 0xFF
    blk[:, :, 1] = sc >> 8
    return blk


def _q4_k_random_blocks(M, K, seed):
    """Random valid Q4_K super-blocks (d, dmin small positive f16; random 6-bit scales and nibbles)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    blk = rng.integers(0, 256, (M, K // 256, 144), dtype=np.uint8)
    for off, scale in ((0, 0.002), (2, 0.001)):
        v = (np.abs(rng.normal(0, scale, (M, K // 256))) + 1e-4).astype(np.float16).view(np.uint16)
        blk[:, :, off] = v & 0xFF
        blk[:, :, off + 1] = v >> 8
    return blk


def _cpu_matmul_leg(blocks, xq, xs, N, M, K, algo):
    """The oracle's matmul (the reference's portable x86 path: per-row block-ordered f32 sums, rows
    split over threads as inference.rs:1318-1330 does) on the same weights and activations, on
    HOST_THREADS and on the reference's default 4 threads; GB/s of the same algorithmic bytes."""
    from oracle import oracle as O
    out = {}
    for nt in sorted({HOST_THREADS, 4}):
        t = time.perf_counter()
        reps = 0
        while reps < 1 or time.perf_counter() - t < 0.2:
            O.matmul_q4_0(xq, xs, blocks, N, M, K, nthreads=nt)
            reps += 1
        dt = (time.perf_counter() - t) / reps
        out[f"{nt}_threads_GBps"] = round(algo / dt / 1e9, 2)
    return out


def run_gemm_sweep(args):
    """Config 1: per-shape median kernel time (dispatch-stamped events around each of >= 60
    back-to-back launches) rotating >= 1 GB of distinct weight copies."""
    import ctypes as C

    import numpy as np
    import torch

    import nanocamelid_amd as nc
    ctx = make_ctx(nc)
    shapes = [(4096, 4096, "q/o"), (1024, 4096, "k/v"), (14336, 4096, "gate/up"), (4096, 14336, "down"),
              (128256, 4096, "lm_head")]
    stream = torch.cuda.current_stream()
    for M, K, name in shapes:
        blocks = _q4_0_random_blocks(M, K, M + K)
        wbytes = M * K // 32 * 18
        copies = max(2, int(np.ceil(1.0e9 / wbytes)))
        mats = [nc.QMat(ctx, nc.NC_TYPE_Q4_0, M, K, blocks) for _ in range(copies)]
        res = {"shape": f"{M}x{K}", "role": name, "weight_bytes": wbytes, "copies": copies}
        handles = (C.c_void_p * copies)(*[m.h for m in mats])
        for N in (1, 2, 5, 9, 16):
            rng = np.random.default_rng(N)
            xq = torch.from_numpy(rng.integers(-127, 128, (N, K), dtype=np.int8)).cuda()
            xs = torch.from_numpy(rng.uniform(0.005, 0.02, (N, K // 32)).astype(np.float32)).cuda()
            out = torch.empty((N, M), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            iters = max(60, 2 * copies)
            us = np.zeros(copies + iters, np.float32)
            # the first round over the copies is warmup; the median is over the next iters launches
            nc.check(nc.lib().nc_bench_matmul(ctx.h, handles, copies, xq.data_ptr(), xs.data_ptr(), out.data_ptr(), N,
                                              copies + iters, us.ctypes.data))
            med = float(np.median(us[copies:]))
            algo = wbytes + N * K + 4 * N * (K // 32) + 4 * N * M
            res[f"N{N}"] = {"us_median": round(med, 2), "GBps": round(algo / med / 1e3, 1),
                            "us_mean": round(float(np.mean(us[copies:])), 2)}
            if not args.no_cpu_baseline:
                res[f"N{N}"]["cpu"] = _cpu_matmul_leg(blocks, xq.cpu().numpy(), xs.cpu().numpy(), N, M, K, algo)
        print(json.dumps(res), flush=True)
        for m in mats:
            m.close()


def run_q4k_sweep(args):
    """The 3B Q4_K layer matrices in isolation: per-shape median kernel time at N = 1, 5, 9
    (dispatch-stamped events, >= 60 launches over >= 1 GB of weight copies).  The kernel variant
    follows the environment (NC_Q4K_PS=<1..4>: pair-split with that many quad lanes)."""
    import ctypes as C

    import numpy as np
    import torch

    import nanocamelid_amd as nc
    ctx = make_ctx(nc)
    res = {"variant": os.environ.get("NC_Q4K_PS", "one wave per quad")}
    for M, K, name in [(5120, 3072, "q,k,v"), (3072, 3072, "wo"), (3072, 8192, "down")]:
        blocks = _q4_k_random_blocks(M, K, M + K)
        wbytes = M * K // 256 * 144
        copies = max(2, int(np.ceil(1.0e9 / wbytes)))
        mats = [nc.QMat(ctx, nc.NC_TYPE_Q4_K, M, K, blocks) for _ in range(copies)]
        handles = (C.c_void_p * copies)(*[m.h for m in mats])
        for N in (1, 5, 9):
            rng = np.random.default_rng(N)
            xq = torch.from_numpy(rng.integers(-127, 128, (N, K), dtype=np.int8)).cuda()
            xs = torch.from_numpy(rng.uniform(0.005, 0.02, (N, K // 32)).astype(np.float32)).cuda()
            out = torch.empty((N, M), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            iters = max(60, 2 * copies)
            us = np.zeros(copies + iters, np.float32)
            nc.check(nc.lib().nc_bench_matmul(ctx.h, handles, copies, xq.data_ptr(), xs.data_ptr(), out.data_ptr(), N,
                                              copies + iters, us.ctypes.data))
            med = float(np.median(us[copies:]))
            res[f"{name} {M}x{K} N{N}"] = {"us_median": round(med, 2), "GBps": round(wbytes / med / 1e3, 1)}
        for m in mats:
            m.close()
    print(json.dumps(res), flush=True)


def run_prefill(args):
    """Prompt prefill (the reference's prefill_tokens, main.rs:9415-9485): (1) the prompt matmul
    alone on the 8B and 70B Q4_0 and 3B Q4_K shapes at 64 and 256 tokens, median of events,
    against the int8 MFMA peak; (2) wall time of an 8B-shape prefill of 512, 2048 and 8192
    tokens in prompt passes, beside the same prompt in 16-token verify-sized passes, whose
    last-row logits must be the same bits."""
    import ctypes as C

    import numpy as np
    import torch

    import nanocamelid_amd as nc
    ctx = make_ctx(nc)
    shapes = [(6144, 4096, "8b q,k,v", 2), (4096, 4096, "8b wo", 2), (28672, 4096, "8b gate,up", 2),
              (4096, 14336, "8b down", 2), (57344, 8192, "70b gate,up", 2), (8192, 28672, "70b down", 2),
              (8192, 3072, "3b Q4_K gate", 12), (3072, 8192, "3b Q4_K down", 12)]
    for M, K, name, ty in (shapes if not args.prefill_tokens else []):
        blocks = _q4_0_random_blocks(M, K, M + K) if ty == 2 else _q4_k_random_blocks(M, K, M + K)
        q = nc.QMat(ctx, ty, M, K, blocks)
        handles = (C.c_void_p * 1)(q.h)
        res = {"shape": f"{M}x{K}", "role": name}
        for N in (64, 256):
            rng = np.random.default_rng(N)
            xq = torch.from_numpy(rng.integers(-127, 128, (N, K), dtype=np.int8)).cuda()
            xs = torch.from_numpy(rng.uniform(0.005, 0.02, (N, K // 32)).astype(np.float32)).cuda()
            out = torch.empty((N, M), dtype=torch.float32, device="cuda")
            us = np.zeros(23, np.float32)
            nc.check(nc.lib().nc_bench_matmul(ctx.h, handles, 1, xq.data_ptr(), xs.data_ptr(), out.data_ptr(), N,
                                              len(us), us.ctypes.data))
            med = float(np.median(us[3:]))
            tops = 2.0 * M * K * N / med / 1e6
            res[f"N{N}"] = {"us_median": round(med, 1), "int8_TOPs": round(tops, 1),
                            "frac_int8_mfma_peak": round(tops / PEAK_INT8_TOPS, 4)}
        q.close()
        print(json.dumps(res), flush=True)
    t0 = time.time()
    img = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3-8b"], context_length=8192 + 64, seed=args.seed,
                        nthreads=HOST_THREADS)
    model = nc.Model(ctx, data=img, nthreads=HOST_THREADS)
    log(f"llama-3-8b-shape model on device in {time.time() - t0:.1f}s")
    prompt = nc.uniform_prompt(args.seed, 8192, model.config["vocab_size"])
    for n in ((args.prefill_tokens,) if args.prefill_tokens else (512, 2048, 8192)):
        s = nc.Session(model, 8192 + 64, 16)
        s.prefill_pass_batch(prompt[:64], 0, want_logits=False)  # the prompt buffers, allocated once
        torch.cuda.synchronize()
        t = time.perf_counter()
        s.prefill_pass_batch(prompt[:n], 0)
        torch.cuda.synchronize()
        tp = time.perf_counter() - t
        res = {"prefill_tokens": n, "prompt_passes_ms": round(tp * 1e3, 1), "prompt_passes_tok_s": round(n / tp)}
        if n <= 2048 and not args.prefill_tokens:
            s2 = nc.Session(model, 8192 + 64, 16)
            t = time.perf_counter()
            for i in range(0, n, 16):
                s2.prefill_pass_batch(prompt[i:i + 16], i, want_logits=(i + 16 >= n))
            torch.cuda.synchronize()
            t16 = time.perf_counter() - t
            res["16_token_passes_ms"] = round(t16 * 1e3, 1)
            res["16_token_passes_tok_s"] = round(n / t16)
            res["last_logits_bit_equal"] = bool(np.array_equal(s.logits(15).view(np.uint32),
                                                               s2.logits(15).view(np.uint32)))
            s2.close()
        s.close()
        print(json.dumps(res), flush=True)
    if not args.no_cpu_baseline and not args.prefill_tokens:
        # the oracle (C++ restatement of the reference's portable path) prefilling the same
        # model: a bounded sample of 64 tokens in the reference's 16-row passes
        from oracle import oracle as O
        om = O.Model(data=img.tobytes(), nthreads=HOST_THREADS)
        n = 64
        s = O.Session(om, n + 16, 16)
        t = time.perf_counter()
        for i in range(0, n, 16):
            s.prefill_pass_batch(prompt[i:i + 16], i)
        dt = time.perf_counter() - t
        s.close()
        om.close()
        print(json.dumps({"cpu_baseline": {"value": round(n / dt, 2), "unit": "prefill tok/s", "cores": HOST_THREADS,
                                           "kind": "port", "cpu_model": cpu_model_name(),
                                           "sample": f"{n}-token prefill of the same llama-3-8b-shape model in "
                                                     f"16-row passes on {HOST_THREADS} threads"}}), flush=True)
    del img


def run_loader(args):
    """GGUF load (gguf.rs:454-551 read_file, model.rs:461-545 LlamaWeights::load, with
    validate_model_tensors model.rs:851-1036): the 8B-shape synthetic file from disk to a model
    ready to run, on the GPU path (mmap, validation, f32 decode of the embedding, repack, upload)
    and in the CPU oracle (its own reader and decode of the same file)."""
    import tempfile

    import nanocamelid_amd as nc
    from oracle import oracle as O
    img = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3-8b"], context_length=8192, seed=args.seed, nthreads=HOST_THREADS)
    size = img.nbytes
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        path = os.path.join(d, "llama-3-8b-q4_0.gguf")
        img.tofile(path)
        del img
        ctx = make_ctx(nc)
        t = time.perf_counter()
        m = nc.Model(ctx, path=path, nthreads=HOST_THREADS)
        ctx.synchronize()
        gpu_s = time.perf_counter() - t
        dev_bytes = int(m.config["device_weight_bytes"])
        m.close()
        t = time.perf_counter()
        om = O.Model(path=path, nthreads=HOST_THREADS)
        cpu_s = time.perf_counter() - t
        om.close()
    print(json.dumps({"metric": "GGUF model load, file to ready model (llama-3-8b shape, Q4_0)", "value": round(gpu_s, 3),
                      "unit": "s", "higher_is_better": False, "file_bytes": int(size), "device_bytes": dev_bytes,
                      "file_GB_per_s": round(size / gpu_s / 1e9, 2),
                      "cpu_baseline": {"value": round(cpu_s, 3), "unit": "s", "cores": HOST_THREADS, "kind": "port",
                                       "sample": "the oracle's load of the same file"}}), flush=True)


def run_config3(args):
    """Config 3: Llama-3.2-3B-shape Q4_K target (tied head requantised to Q4_0), Llama-3.2-1B-shape
    Q4_0 draft, temperature 1.0, k=4, Philox min(1, p/q) acceptance, 4096-position context.
    One timed call of the device decode loop after a short warmup call; prints one JSON line."""
    import numpy as np
    import torch

    import nanocamelid_amd as nc
    t0 = time.time()
    timg = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3.2-3b-q4k"], context_length=8192, seed=args.seed,
                         nthreads=HOST_THREADS)
    dimg = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3.2-1b"], context_length=8192, seed=args.seed + 1,
                         nthreads=HOST_THREADS)
    log(f"synthetic target {timg.nbytes / 1e9:.2f} GB + draft {dimg.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    ctx = make_ctx(nc)
    tm = nc.Model(ctx, data=timg, nthreads=HOST_THREADS)
    dm = nc.Model(ctx, data=dimg, nthreads=HOST_THREADS)
    V = tm.config["vocab_size"]
    n_prompt, max_ctx = args.c3_prompt, 4096
    n_new = min(args.c3_new, max_ctx - n_prompt - args.k - 2)
    prompt = nc.uniform_prompt(args.seed, n_prompt, V)
    temp = 1.0

    def run(n, timing=False):
        ts, ds = nc.Session(tm, max_ctx, 16), nc.Session(dm, max_ctx, 16)
        ts.timing(timing)
        out, st = nc.generate_speculative_stochastic(ts, ds, prompt, n, args.k, temp, args.seed)
        gt = ts.gemm_timing() if timing else (0, 0.0, 0)
        ts.close()
        ds.close()
        return out, st, gt

    run(64)  # warmup
    torch.cuda.synchronize()
    out, st, _ = run(n_new)
    tok = st.emitted - 1  # the first token comes from the prompt pass
    tok_s = tok / st.decode_seconds
    log(f"config 3: {st.steps} steps, {tok} tokens in {st.decode_seconds:.3f}s = {tok_s:.1f} tok/s, acceptance "
        f"{st.accepted}/{st.drafted}, prefill {st.prefill_seconds:.2f}s")
    _, _, (launches, gemm_ms, gemm_bytes) = run(min(n_new, 256), timing=True)
    achieved = gemm_bytes / (gemm_ms / 1e3) / 1e9 if launches else 0.0
    log(f"target gemm: {launches} launches, {gemm_ms / max(launches, 1) * 1e3:.2f} us avg -> {achieved:.0f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        tmo, dmo = O.Model(data=timg.tobytes(), nthreads=HOST_THREADS), O.Model(data=dimg.tobytes(), nthreads=HOST_THREADS)
        cp = prompt[:16]
        tp = time.time()
        O.generate_speculative_stochastic(O.Session(tmo, 256, 16), O.Session(dmo, 256, 16), cp, 1, args.k, temp, args.seed)
        t_prefill = time.time() - tp
        td = time.time()
        o, drafted, accepted, nsteps = O.generate_speculative_stochastic(O.Session(tmo, 256, 16), O.Session(dmo, 256, 16),
                                                                         cp, 1 + args.cpu_steps * (args.k + 1), args.k,
                                                                         temp, args.seed)
        t_dec = time.time() - td - t_prefill
        cpu = {"value": round((len(o) - 1) / t_dec, 4), "unit": "tok/s", "cores": HOST_THREADS, "kind": "port",
               "sample": f"same models on the host: 16-token prompt, {nsteps} stochastic steps (k={args.k}, T=1.0, "
                         f"{len(o) - 1} tokens, {accepted}/{drafted} accepted) in {t_dec:.1f}s"}
        log(f"cpu baseline: {cpu}")
    line = {
        "metric": "verified tok/s (config 3: Llama-3.2-3B-shape Q4_K target, 1B-shape Q4_0 draft, T=1.0, k=4, "
                  "Philox acceptance)",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": int(st.steps), "warmup": 1,
        "ms_per_step": round(st.decode_seconds / max(st.steps, 1) * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8 dot -> int32, f32 accumulate",
        "data": "synthetic (random-init weights N(0,0.02) -> Q4_K / Q4_0, seeded uniform prompt)",
        "config": {"workload": f"llama-3.2-3b-q4k target + llama-3.2-1b draft, stochastic speculative sampling k={args.k} "
                               f"T=1.0, {n_prompt}-token prompt, {int(tok)} new tokens, 4096-position KV",
                   "gemm_kernel": GEMM_KERNEL, "attention": ATTENTION, "pass_launch": PASS_LAUNCH,
                   "k": args.k, "temperature": temp, "prompt_tokens": n_prompt, "tokens_emitted": int(tok),
                   "drafted": int(st.drafted), "accepted": int(st.accepted),
                   "target_verify_weight_bytes": int(tm.config["verify_weight_bytes"]),
                   "draft_weight_bytes": int(dm.config["verify_weight_bytes"])},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "target verify matmuls (gemm_q4_k_r16_kernel q,k,v, wo, down + gemm_q4_k_ps_kernel gate,up + gemm_q4_0_kernel head)",
                     "launches": int(launches), "avg_us": round(gemm_ms / max(launches, 1) * 1e3, 3),
                     "avg_algorithmic_bytes": int(gemm_bytes // max(launches, 1))},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_config4(args):
    """Config 4: Llama-3-70B-shape Q4_0 (untied head), one k+1 = 9-row verify pass over an
    8192-position KV cache filled with N(0, 1) keys and values (nc_session_fill_kv: seeded
    Philox + Box-Muller streams, the same values the oracle's or_session_fill_kv draws).
    value = verify passes per second (timed passes re-verify the same 9 positions, whose KV rows
    each pass rewrites identically).  Checks: drafts equal to the greedy continuation (single-token
    passes from position 8192) are all accepted; and the CPU leg, one 9-row pass of the oracle on
    the whole model over the same filled cache, must give every row's logits bit for bit."""
    import numpy as np
    import torch

    import nanocamelid_amd as nc
    t0 = time.time()
    img = nc.synth_gguf(**nc.SYNTH_CONFIGS["llama-3-70b"], context_length=8192 + 64, seed=args.seed,
                        nthreads=HOST_THREADS)
    log(f"synthetic llama-3-70b GGUF: {img.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    ctx = make_ctx(nc)
    t0 = time.time()
    model = nc.Model(ctx, data=img, nthreads=HOST_THREADS)
    if args.no_cpu_baseline:
        del img
    cfg = model.config
    log(f"model on device in {time.time() - t0:.1f}s: {cfg['verify_weight_bytes'] / 1e9:.2f} GB streamed per verify")
    n_ctx, n = 8192, 9
    sess = nc.Session(model, n_ctx + 64, 16)
    t0 = time.time()
    sess.fill_kv(n_ctx, args.seed)
    fill_s = time.time() - t0
    log(f"N(0, 1) fill of {n_ctx} KV positions in {fill_s:.1f}s")
    # greedy continuation of n tokens at positions n_ctx.. (single-token passes)
    greedy = [int(nc.uniform_prompt(args.seed, 1, cfg["vocab_size"])[0])]
    for i in range(n - 1):
        nxt, _ = sess.forward_pass(greedy[-1], n_ctx + i, want_logits=False)
        greedy.append(nxt)
    batch = np.array(greedy, np.uint32)  # [pending] + 8 drafts = the greedy continuation
    a, nxt, newpos, preds = sess.verify_greedy(batch, n_ctx)
    consistent = bool(a == n - 1 and np.array_equal(preds[:n - 1], batch[1:]))
    log(f"verify of the greedy continuation: accepted {a}/{n - 1}, consistent with single-token passes: {consistent}")
    for _ in range(2):
        sess.verify_greedy(batch, n_ctx)
    torch.cuda.synchronize()
    sess.timing(True)
    t0 = time.time()
    reps = args.c4_passes
    for _ in range(reps):
        sess.verify_greedy(batch, n_ctx)
    torch.cuda.synchronize()
    dt = (time.time() - t0) / reps
    launches, gemm_ms, gemm_bytes = sess.gemm_timing()
    sess.timing(False)
    achieved = gemm_bytes / (gemm_ms / 1e3) / 1e9
    kv_bytes = 2 * cfg["block_count"] * cfg["kv_width"] * (n_ctx + n) * 4
    log(f"verify pass: {dt * 1e3:.2f} ms ({(cfg['verify_weight_bytes'] + kv_bytes) / dt / 1e9:.0f} GB/s incl. KV); "
        f"matmuls {gemm_ms / reps:.2f} ms -> {achieved:.0f} GB/s")
    gpu_logits = [sess.logits(i) for i in range(n)]
    if args.copy_calibration:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 256 MiB device-to-device copies")
    cpu, parity = None, None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        t0 = time.time()
        om = O.Model(data=img, nthreads=HOST_THREADS)
        os_ = O.Session(om, n_ctx + 64, 16)
        os_.fill_kv(n_ctx, args.seed)
        log(f"oracle: model and N(0, 1) fill in {time.time() - t0:.1f}s; one 9-row verify pass on {HOST_THREADS} threads")
        t0 = time.perf_counter()
        opreds, _, ologits = os_.verify_greedy(batch, n_ctx, want_logits=True)
        cpu_s = time.perf_counter() - t0
        same = [bool(np.array_equal(gpu_logits[i].view(np.uint32), ologits[i].view(np.uint32))) for i in range(n)]
        parity = {"rows_bit_identical": int(sum(same)), "rows": n,
                  "preds_identical": bool(np.array_equal(preds, opreds))}
        log(f"oracle verify pass {cpu_s:.1f}s; logits bit-identical on {sum(same)}/{n} rows")
        cpu = {"value": round(1.0 / cpu_s, 5), "unit": "verify passes/s", "cores": HOST_THREADS, "kind": "port",
               "cpu_model": cpu_model_name(), "nproc": os.cpu_count(),
               "sample": "one 9-row verify pass of the same llama-3-70b-shape model over the same 8192 N(0, 1) "
                         f"KV positions (the oracle, {HOST_THREADS} threads)", "seconds": round(cpu_s, 2)}
        os_.close()
        om.close()
        del img
    line = {
        "metric": "verify pass time (config 4: Llama-3-70B-shape Q4_0, 9 rows, 8192-position KV)",
        "value": round(1.0 / dt, 3), "unit": "verify passes/s", "n_gpus": 1, "steps": reps, "warmup": 2,
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 dot -> int32, f32 accumulate",
        "data": "synthetic (random-init weights N(0,0.02) -> Q4_0; KV cache of 8192 positions of N(0, 1) keys and "
                "values from seeded Philox + Box-Muller streams)",
        "config": {"workload": "llama-3-70b-shape Q4_0 single k+1 verify (k=8) over an 8192-position KV cache",
                   "gemm_kernel": GEMM_KERNEL, "attention": ATTENTION, "pass_launch": PASS_LAUNCH,
                   "rows": n, "kv_positions": n_ctx, "verify_weight_bytes": int(cfg["verify_weight_bytes"]),
                   "kv_bytes_read": int(kv_bytes), "greedy_drafts_all_accepted": consistent,
                   "kv_fill_s": round(fill_s, 2), "oracle_parity": parity},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": _traffic_from(TRAFFIC_PROFILE_C4),
                     "kernel": "gemm_q4_0_kernel / gemm_q4_0_r16_kernel (all verify matmuls)",
                     "launches": int(launches), "avg_us": round(gemm_ms / max(launches, 1) * 1e3, 3),
                     "avg_algorithmic_bytes": int(gemm_bytes // max(launches, 1))},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="llama-3-8b")
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--alpha", type=float, default=0.8)
    ap.add_argument("--n-prompt", type=int, default=512)
    ap.add_argument("--n-new", type=int, default=1024)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--roofline-steps", type=int, default=40)
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-full-decode", action="store_true", help="skip the 1024-token decodes at each (k, alpha)")
    ap.add_argument("--gemm-sweep", action="store_true", help="config 1: isolated GEMM bandwidth table")
    ap.add_argument("--q4k-sweep", action="store_true", help="config 3's Q4_K layer matrices in isolation")
    ap.add_argument("--config3", action="store_true",
                    help="config 3: 3B Q4_K target + 1B Q4_0 draft, stochastic acceptance (T=1, k=4)")
    ap.add_argument("--config4", action="store_true",
                    help="config 4: 70B Q4_0, one 9-row verify pass over an 8192-position KV cache")
    ap.add_argument("--prefill", action="store_true",
                    help="prompt prefill: prompt matmul at 64/256 tokens and 8B-shape prefill wall times")
    ap.add_argument("--loader", action="store_true", help="GGUF load time from disk (GPU path and CPU oracle)")
    ap.add_argument("--prefill-tokens", type=int, default=0,
                    help="with --prefill: only one prefill of this many tokens (for a kernel profile)")
    ap.add_argument("--c4-passes", type=int, default=10)
    ap.add_argument("--c3-prompt", type=int, default=3072)
    ap.add_argument("--c3-new", type=int, default=768)
    ap.add_argument("--gemm-kernel", choices=sorted(GEMM_KERNELS), default="auto",
                    help="dot-product path of the Q4_0 16-row matmuls (nc_ctx_set_gemm_kernel)")
    ap.add_argument("--attention", choices=sorted(ATTENTION_ORDERS), default="sequential",
                    help="summation order of the verify passes' attention (nc_ctx_set_attention)")
    ap.add_argument("--no-split-report", action="store_true",
                    help="skip the extra run of the opt-in split-position attention")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 256 MiB device copy (known HBM bytes) to scale rocprofv3 --pmc byte counters")
    ap.add_argument("--pass-launch", choices=sorted(PASS_LAUNCHES), default="direct",
                    help="verify/decode passes replayed from HIP graphs or launched kernel by kernel "
                         "(nc_ctx_set_pass_launch)")
    args = ap.parse_args()
    global GEMM_KERNEL, ATTENTION, PASS_LAUNCH
    GEMM_KERNEL = args.gemm_kernel
    ATTENTION = args.attention
    PASS_LAUNCH = args.pass_launch
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU (multi-GPU sharding is designed, not "
                                   "built); run with --gpus 1"}))
        sys.exit(2)

    import numpy as np
    import torch

    import nanocamelid_amd as nc

    assert torch.cuda.is_available(), "bench needs the MI355X"
    if args.q4k_sweep:
        run_q4k_sweep(args)
        return
    if args.gemm_sweep:
        run_gemm_sweep(args)
        return
    if args.config3:
        run_config3(args)
        return
    if args.config4:
        run_config4(args)
        return
    if args.prefill:
        run_prefill(args)
        return
    if args.loader:
        run_loader(args)
        return
    spec = dict(nc.SYNTH_CONFIGS[args.config])
    t0 = time.time()
    img = nc.synth_gguf(**spec, context_length=8192, seed=args.seed, nthreads=HOST_THREADS)
    log(f"synthetic {args.config} GGUF: {img.nbytes / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    ctx = make_ctx(nc)
    t0 = time.time()
    model = nc.Model(ctx, data=img, nthreads=HOST_THREADS)
    cfg = model.config
    log(f"model on device in {time.time() - t0:.1f}s: {cfg['device_weight_bytes'] / 1e9:.3f} GB repacked, "
        f"{cfg['verify_weight_bytes'] / 1e9:.3f} GB streamed per verify")
    prompt = nc.uniform_prompt(args.seed, args.n_prompt, cfg["vocab_size"])
    n_rec = args.n_new + 32 * (args.k + 1)
    max_ctx = args.n_prompt + n_rec + 32
    sess = nc.Session(model, max_ctx, 16)
    t0 = time.time()
    greedy, gst = sess.generate_greedy(prompt, n_rec)
    log(f"greedy record: {n_rec} tokens in {gst.decode_seconds:.2f}s ({n_rec / gst.decode_seconds:.1f} tok/s plain "
        f"greedy), prefill {gst.prefill_seconds:.2f}s")
    ref_order = None
    if ATTENTION != "sequential":
        # the same greedy continuation in the reference's attention order: where does the
        # split order's stream first leave it
        ctx.set_attention(ATTENTION_ORDERS["sequential"])
        rgreedy, _ = nc.Session(model, max_ctx, 16).generate_greedy(prompt, n_rec)
        ctx.set_attention(ATTENTION_ORDERS[ATTENTION])
        div = next((i for i in range(n_rec) if int(rgreedy[i]) != int(greedy[i])), None)
        ref_order = {"tokens": n_rec, "identical": div is None, "first_divergence": div}
        log(f"greedy stream against the reference attention order: {ref_order}")

    # warmup steps (untimed), then exactly K timed steps
    sess.generate_speculative_oracle(prompt, n_rec, args.k, args.alpha, args.seed, greedy, max_steps=args.warmup)
    torch.cuda.synchronize()
    out, st = sess.generate_speculative_oracle(prompt, n_rec, args.k, args.alpha, args.seed, greedy,
                                               max_steps=args.steps)
    torch.cuda.synchronize()
    parity = bool(np.array_equal(out, greedy[:len(out)]))
    emitted_by_steps = st.emitted - 1  # the first token comes from the prefill pass
    tok_s = emitted_by_steps / st.decode_seconds
    log(f"speculative: {st.steps} steps, {emitted_by_steps} tokens in {st.decode_seconds:.3f}s = {tok_s:.1f} tok/s, "
        f"acceptance {st.accepted}/{st.drafted}, stream == greedy: {parity}")

    # roofline pass: HIP events around every verify GEMM launch on the session stream
    # (the prompt prefill inside the call is not timed)
    launches, gemm_ms, gemm_bytes, achieved = 0, 0.0, 0, 0.0
    if args.roofline_steps > 0:
        sess.timing(True)
        sess.generate_speculative_oracle(prompt, n_rec, args.k, args.alpha, args.seed, greedy,
                                         max_steps=args.roofline_steps)
        launches, gemm_ms, gemm_bytes = sess.gemm_timing()
        sess.timing(False)
        achieved = gemm_bytes / (gemm_ms / 1e3) / 1e9
        log(f"gemm: {launches} launches, {gemm_ms / launches * 1e3:.2f} us avg, "
            f"{gemm_bytes / launches / 1e6:.2f} MB avg -> {achieved:.0f} GB/s")
    # stage pass: HIP events between the stages of every verify pass, named as the reference's
    # NANOCAMELID_TRACE stages (inference.rs:179-229); a separate run, outside the timed region
    stages = None
    if args.roofline_steps > 0:
        sess.stage_timing(True)
        _, sst2 = sess.generate_speculative_oracle(prompt, n_rec, args.k, args.alpha, args.seed, greedy,
                                                   max_steps=args.roofline_steps)
        raw = sess.stages()
        sess.stage_timing(False)
        npass = max(sst2.steps, 1)
        per = {k: round(v[0] / npass * 1e3, 2) for k, v in raw.items()}
        total = sum(per.values())
        stages = {"us_per_verify_pass": per, "sum_us": round(total, 1),
                  "share": {k: round(v / total, 4) for k, v in per.items()} if total else {},
                  "passes": int(npass), "calls": {k: int(v[1]) for k, v in raw.items()},
                  "note": "events between stages on the session stream; stage names are the reference's trace "
                          "stages, '+' joins stages the device runs as one kernel"}
        log(f"stages (us per verify pass): {per}")
    # the config's whole 1024-token decode at every (k, alpha) point, each a separate call
    full = {}
    if not args.no_full_decode:
        for k in (2, 4, 8):
            for alpha in (0.5, 0.8):
                o, fs = sess.generate_speculative_oracle(prompt, args.n_new + 1, k, alpha, args.seed, greedy)
                ftok = fs.emitted - 1
                full[f"k{k}_alpha{alpha}"] = {
                    "tok_s": round(ftok / fs.decode_seconds, 2), "tokens": int(ftok), "steps": int(fs.steps),
                    "drafted": int(fs.drafted), "accepted": int(fs.accepted),
                    "positions": f"{args.n_prompt}..{args.n_prompt + ftok}",
                    "stream_equals_greedy": bool(np.array_equal(o, greedy[:len(o)]))}
                log(f"full decode k={k} alpha={alpha}: {full[f'k{k}_alpha{alpha}']}")
    # the opt-in split-position attention on the same model and drafter (not the headline: its
    # arithmetic is not the reference's); where its greedy stream leaves the reference order's
    split = None
    if ATTENTION == "sequential" and not args.no_split_report:
        ctx.set_attention(ATTENTION_ORDERS["split"])
        ss = nc.Session(model, max_ctx, 16)
        sgreedy, _ = ss.generate_greedy(prompt, n_rec)
        ss.generate_speculative_oracle(prompt, n_rec, args.k, args.alpha, args.seed, sgreedy, max_steps=args.warmup)
        torch.cuda.synchronize()
        so, sst = ss.generate_speculative_oracle(prompt, n_rec, args.k, args.alpha, args.seed, sgreedy,
                                                 max_steps=args.steps)
        ss.close()
        ctx.set_attention(ATTENTION_ORDERS["sequential"])
        stok = sst.emitted - 1  # as the headline: the first token comes from the prefill pass
        div = next((i for i in range(n_rec) if int(sgreedy[i]) != int(greedy[i])), None)
        split = {"tok_s": round(stok / sst.decode_seconds, 2), "steps": int(sst.steps), "tokens": int(stok),
                 "stream_equals_its_greedy": bool(np.array_equal(so, sgreedy[:len(so)])),
                 "greedy_first_divergence_from_reference_order": div}
        log(f"split attention (opt-in): {split}")
    # GPU greedy continuation of a 16-token prompt, for the CPU stream comparison
    stream_prompt = prompt[:16]
    s16 = nc.Session(model, 64, 16)
    gpu_stream, _ = s16.generate_greedy(stream_prompt, 9)
    s16.close()
    if args.copy_calibration:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 256 MiB device-to-device copies")

    cpu = None
    tok_per_step = emitted_by_steps / max(st.steps, 1)
    if not args.no_cpu_baseline:
        sess.close()
        model.close()
        cpu = cpu_baseline(img, cfg, args, tok_per_step, gpu_stream, stream_prompt)
        log(f"cpu baseline: {cpu}")

    # whole-pass bytes: verify weights + the K and V rows each step reads once (positions grow
    # linearly from the prompt end over the timed steps, so the mean position is used)
    ms_step = st.decode_seconds / st.steps * 1e3
    kv_step = 2 * cfg["block_count"] * cfg["kv_width"] * 4 * (args.n_prompt + emitted_by_steps / 2 + args.k + 1)
    whole_gbs = (cfg["verify_weight_bytes"] + kv_step) / (ms_step / 1e3) / 1e9
    log(f"whole pass: {(cfg['verify_weight_bytes'] + kv_step) / 1e9:.3f} GB per step (KV {kv_step / 1e6:.0f} MB) "
        f"-> {whole_gbs:.0f} GB/s")
    line = {
        "metric": "verified tok/s (Llama-3-8B Q4_0, k=4) + verify matmul HBM GB/s vs peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": int(st.steps),
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot -> int32, f32 accumulate",
        "data": "synthetic (random-init weights N(0,0.02) -> Q4_0, seeded uniform prompt)",
        "config": {"workload": f"{args.config}-shape Q4_0 greedy speculative decode, oracle drafter k={args.k} "
                               f"alpha={args.alpha}, {args.n_prompt}-token prompt; timed: {st.steps} steps emitting "
                               f"{emitted_by_steps} tokens at positions {args.n_prompt}..{args.n_prompt + emitted_by_steps}"
                               f" (the config's full {args.n_new}-token decode at every k, alpha: full_decode)",
                   "timed_positions": [args.n_prompt, args.n_prompt + emitted_by_steps],
                   "full_decode": full,
                   "gemm_kernel": GEMM_KERNEL, "attention": ATTENTION, "pass_launch": PASS_LAUNCH,
                   "k": args.k, "alpha": args.alpha, "prompt_tokens": args.n_prompt,
                   "tokens_emitted": int(emitted_by_steps), "drafted": int(st.drafted),
                   "accepted": int(st.accepted), "stream_equals_greedy": parity,
                   "greedy_vs_reference_attention_order": ref_order,
                   "opt_in_split_attention": split,
                   "verify_weight_bytes": int(cfg["verify_weight_bytes"]),
                   "kv_bytes_read_per_step": int(kv_step),
                   "whole_pass_GBps": round(whole_gbs, 1),
                   "stages": stages},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": measured_traffic(args),
                     "kernel": "gemm_q4_0_r16_kernel + gemm_q4_0_kernel (all verify matmuls)",
                     "launches": int(launches), "avg_us": round(gemm_ms / max(launches, 1) * 1e3, 3),
                     "avg_algorithmic_bytes": int(gemm_bytes // max(launches, 1))},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
