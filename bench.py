"""Benchmark of the fermix_amd hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line. A "step"
is one pass of the hot path over one batch of synthetic input already resident in HBM:

* the headline workload: fp32 slogpf forward, B = 4096,
  n = 128, S = A - A^T with A iid N(0, 1) from numpy default_rng(0) (jax, whose
  jax.random.key(0) the BASELINE names, is not installed here or on the GPU box);
* reported beside it in "workloads": configs[0] (slogdet forward, B = 4096, n = 128)
  and configs[2] (slogdet forward + VJP, B = 1024, n = 512) when the library supports
  it.

`roofline` is the dominant kernel's algorithmic bytes per launch (B (4 n^2 + 8): read
each matrix once, write sign and logabs) divided by its average launch duration over
the timed region, timed with HIP events on the stream the kernel is launched on.
`cpu_baseline` times the CPU oracle (the reference's generic path restated in numpy,
oracle/generic.py) on a bounded sample of the same workload on this host, rank 0 only:
`value` with one BLAS thread, `value_all_cores` with one single-threaded process per
host CPU (at most 16, the box's CPU share of one GPU), with the CPU model, CPU count and
thread environment beside it. The CPU legs run before the GPU is initialised.
"""

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # 200 timed steps by default: 20-step windows of the n = 128 workloads scatter by
    # 2-4 % with the GPU's clock (0.1745-0.1826 ms/step for C2 in one process)
    p.add_argument("--steps", type=int, default=200)
    # 100 untimed steps by default: after an idle period the GPU's clocks ramp up over the
    # first ~60 steps of the n = 128 workloads (C2 0.1925 -> 0.1813 ms/step over the first
    # 60 steps after 5 warm-up steps), so a short warm-up times the ramp, not the kernel
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--only", default=None, help="comma list of workloads (c1,c2,c3,c4; f64 adds the float64 "
                   "n = 128 workloads, blk the blocked float64 / complex ones at n = 512, xxl the B = 1 "
                   "orders 8192 / 16384, all reported on stderr)")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run a plain 256 MiB device copy (calibrates FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


HEAD_KERNEL = {"slogpf_fwd": "pf_small_kernel<128, false>", "slogdet_fwd": "lu_split_kernel<128, 64, false>"}


def _measured_traffic(name):
    """HBM bytes per dispatch of the workload's kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/traffic.txt), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.txt")
    kern = HEAD_KERNEL.get(name)
    if kern is None or not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(kern + " "):
            return int(line.split()[-1])
    return None


def _time_gpu(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / steps, wall


def _inputs(B, n, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((B, n, n), dtype=np.float32)
    if scale != 1.0:
        A *= np.float32(scale)
    return A


def bench_c2(steps, warmup, skew_symmetrize=True):
    """slogpf forward, B = 4096, n = 128, S = A - A^T. The headline calls the
    API default (skew_symmetrize=True, fused into the kernel's load; (S - S^T) / 2 = S
    bitwise here); skew_symmetrize=False is reported beside it."""
    import torch
    import fermix_amd

    B, n = 4096, 128
    A = _inputs(B, n, 0)
    S = torch.from_numpy(A - np.swapaxes(A, 1, 2)).cuda()
    fn = lambda: fermix_amd.slogpf(S, skew_symmetrize=skew_symmetrize)
    ms, wall = _time_gpu(fn, steps, warmup)
    name = "slogpf_fwd" if skew_symmetrize else "slogpf_fwd_noskew"
    return dict(name=name, B=B, n=n, ms=ms, wall=wall, rate=B / (ms * 1e-3),
                bytes=B * (4 * n * n + 8), sample=S[:64].cpu().numpy())


def bench_c1(steps, warmup):
    import torch
    import fermix_amd

    B, n = 4096, 128
    A = torch.from_numpy(_inputs(B, n, 0)).cuda()
    fn = lambda: fermix_amd.slogdet(A)
    ms, wall = _time_gpu(fn, steps, warmup)
    return dict(name="slogdet_fwd", B=B, n=n, ms=ms, wall=wall, rate=B / (ms * 1e-3),
                bytes=B * (4 * n * n + 8), sample=A[:64].cpu().numpy())


def bench_c3(steps, warmup, prec=None):
    """slogdet forward + VJP (cotangent ones on logabs), B = 1024, n = 512,
    A iid N(0, 1/n); prec None (the API default, "bf16x3" for float32) or "ieee" (fp32
    MFMA)."""
    import torch
    import fermix_amd

    B, n = 1024, 512
    A = torch.from_numpy(_inputs(B, n, 0, scale=1.0 / np.sqrt(n))).cuda().requires_grad_()

    def fn():
        s, l = fermix_amd.slogdet(A, prec=prec)
        (g,) = torch.autograd.grad(l.sum(), A)
        return g

    ms, wall = _time_gpu(fn, steps, warmup)
    name = "slogdet_fwd_grad" + ("" if prec is None else "_" + prec)
    return dict(name=name, B=B, n=n, ms=ms, wall=wall, rate=B / (ms * 1e-3),
                bytes=B * 8 * n * n, flops=B * 2.0 * n ** 3, sample=None)


def bench_c4(steps, warmup, prec=None):
    """slogpf forward + VJP (cotangent ones on log|pf|), B = 64, n = 2048,
    S = A - A^T with A iid N(0, 1/n), called with the API defaults (skew_symmetrize=True,
    whose (S - S^T) / 2 = S, and prec None: "bf16x3") or prec "ieee"."""
    import torch
    import fermix_amd

    B, n = 64, 2048
    A = _inputs(B, n, 0, scale=1.0 / np.sqrt(n))
    S = torch.from_numpy(A - np.swapaxes(A, 1, 2)).cuda().requires_grad_()
    del A

    def fn():
        s, l = fermix_amd.slogpf(S, prec=prec)
        (g,) = torch.autograd.grad(l.sum(), S)
        return g

    ms, wall = _time_gpu(fn, steps, warmup)
    name = "slogpf_fwd_grad" + ("" if prec is None else "_" + prec)
    return dict(name=name, B=B, n=n, ms=ms, wall=wall, rate=B / (ms * 1e-3),
                bytes=B * 8 * n * n, flops=B * 1.0 * n ** 3, sample=None)


def _oracle_fn(which):
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import generic as g

    return g.slogpf_generic if which == "slogpf" else g.slogdet_generic


def _cpu_worker(args):
    """One process of the all-core leg: the oracle on its slice for about `secs` seconds,
    one BLAS thread; returns (matrices done, seconds)."""
    sample, which, secs = args
    from threadpoolctl import threadpool_limits

    f = _oracle_fn(which)
    with threadpool_limits(limits=1):
        f(sample[:1])
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < secs:
            f(sample)
            done += sample.shape[0]
    return done, time.perf_counter() - t0


def cpu_baseline(sample, which, workers):
    """The CPU oracle on a bounded sample: one thread (matrices/s), then `workers`
    processes of one thread each over slices of the sample (the all-core figure)."""
    from concurrent.futures import ProcessPoolExecutor

    done, t = _cpu_worker((sample, which, 10.0))
    one = done / t
    reps = done // sample.shape[0]
    allc = None
    if workers > 1:
        parts = [sample[i::workers] for i in range(workers)]
        parts = [p for p in parts if p.shape[0]]
        with ProcessPoolExecutor(len(parts)) as ex:
            res = list(ex.map(_cpu_worker, [(p, which, 8.0) for p in parts]))
        allc = sum(d for d, _ in res) / max(tt for _, tt in res)
    return one, reps, t, allc


def host_info():
    """CPU model, logical CPU count and the thread environment of this host."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    env = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS",
                                          "XLA_FLAGS") if os.environ.get(k) is not None}
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = None
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": aff, "thread_env": env}


def cpu_library():
    """numpy.linalg.slogdet (LAPACK getrf per matrix) on the full C1 batch on the host cores:
    the CPU library figure beside the oracle port (jax, whose jnp.linalg.slogdet the
    reference would time, is not installed). One thread, then up to 16 (the box's CPU
    share for one GPU). Returns {threads: matrices/s}."""
    from threadpoolctl import threadpool_limits

    A = _inputs(4096, 128, 0)
    out = {}
    for threads in (1, min(16, os.cpu_count() or 1)):
        with threadpool_limits(limits=threads):
            np.linalg.slogdet(A[:64])
            reps, t, t0 = 0, 0.0, time.perf_counter()
            while t < 3.0:
                np.linalg.slogdet(A)
                reps += 1
                t = time.perf_counter() - t0
        out[threads] = A.shape[0] * reps / t
    return out


def bench_f64(steps, warmup):
    """float64 counterparts of the n = 128 workloads (B = 4096, the C1 / C2 inputs in
    float64): slogpf and slogdet forward, and slogdet forward + gradient; and the slogdet
    forward at n = 16 / 32, B = 65536, beside torch.linalg.slogdet."""
    import torch
    import fermix_amd

    B, n = 4096, 128
    A64 = _inputs(B, n, 0).astype(np.float64)
    A = torch.from_numpy(A64).cuda()
    S = torch.from_numpy(A64 - np.swapaxes(A64, 1, 2)).cuda()
    Ag = A.clone().requires_grad_()

    def grad():
        s, l = fermix_amd.slogdet(Ag)
        (g,) = torch.autograd.grad(l.sum(), Ag)
        return g

    out = {}
    for name, fn, nbytes in [
        ("f64_slogpf_fwd", lambda: fermix_amd.slogpf(S, skew_symmetrize=False), 8 * n * n + 16),
        ("f64_slogdet_fwd", lambda: fermix_amd.slogdet(A), 8 * n * n + 16),
        ("f64_slogdet_fwd_grad", grad, 16 * n * n),
    ]:
        ms, wall = _time_gpu(fn, steps, warmup)
        out[name] = dict(name=name, B=B, n=n, ms=ms, wall=wall, rate=B / (ms * 1e-3),
                         bytes=B * nbytes, sample=None)
    # small orders, several matrices per wave, beside torch.linalg.slogdet (rocSOLVER)
    for n_small in (16, 32):
        Bs = 65536
        As = torch.from_numpy(_inputs(Bs, n_small, 2).astype(np.float64)).cuda()
        for name, fn in [(f"f64_slogdet_fwd_n{n_small}", lambda: fermix_amd.slogdet(As)),
                         (f"torch_f64_slogdet_fwd_n{n_small}", lambda: torch.linalg.slogdet(As))]:
            ms, wall = _time_gpu(fn, steps, warmup)
            out[name] = dict(name=name, B=Bs, n=n_small, ms=ms, wall=wall, rate=Bs / (ms * 1e-3),
                             bytes=Bs * (8 * n_small * n_small + 16), sample=None)
        del As
    return out


def bench_blocked(steps, warmup):
    """The blocked float64 / complex kernels (lu64_impl.inc) at B = 32, n = 512: the value
    and gradient factors (sign, logabs and A^-T or S^-1) of slogdet and slogpf in float64,
    complex64 (both product modes) and complex128, on the C3-shaped inputs (complex: a
    second draw as the imaginary part)."""
    import torch
    from fermix_amd import _kernels

    B, n = 32, 512
    re = _inputs(B, n, 0).astype(np.float64)
    im = _inputs(B, n, 1).astype(np.float64)
    out = {}
    for kind, arr in [("f64", re), ("c64", (re + 1j * im).astype(np.complex64)),
                      ("c128", re + 1j * im)]:
        A = torch.from_numpy(np.ascontiguousarray(arr)).cuda()
        S = (A - A.transpose(1, 2)).contiguous()
        esz = A.element_size()
        runs = [(f"blk_{kind}_slogdet_parts", lambda: _kernels.slogdet_parts(A)),
                (f"blk_{kind}_slogpf_parts", lambda: _kernels.slogpf_parts(S, False))]
        if kind == "c64":  # complex64's fp32-product mode beside the default
            runs += [("blk_c64_ieee_slogdet_parts", lambda: _kernels.slogdet_parts(A, x3=0)),
                     ("blk_c64_ieee_slogpf_parts", lambda: _kernels.slogpf_parts(S, False, x3=0))]
        for name, fn in runs:
            ms, wall = _time_gpu(fn, steps, warmup)
            out[name] = dict(name=name, B=B, n=n, ms=ms, wall=wall, rate=B / (ms * 1e-3),
                             bytes=B * 2 * esz * n * n, sample=None)
        del A, S
    return out


def bench_xxl(steps, warmup):
    """B = 1 at the largest orders: float32 n = 8192 (its own blocked kernels) and
    n = 16384 (the field-generic blocked kernels on float storage), float64 and complex128
    at n = 8192: slogdet and slogpf forwards and the parts runs (with A^-T / S^-1) of
    I + N(0, 1/(4n)) (complex: both parts), inputs generated on the GPU."""
    import torch
    from fermix_amd import _kernels

    out = {}
    for kind, n in [("f32", 8192), ("f32", 16384), ("f64", 8192), ("c128", 8192)]:
        dt = {"f32": torch.float32, "f64": torch.float64, "c128": torch.complex128}[kind]
        g = torch.Generator(device="cuda").manual_seed(n)
        A = torch.randn((1, n, n), generator=g, dtype=dt, device="cuda") * (0.5 / np.sqrt(n))
        A.diagonal(dim1=1, dim2=2).add_(1.0)
        S = (A - A.transpose(1, 2)).contiguous()
        esz = A.element_size()
        for name, fn in [(f"xxl_{kind}_{n}_slogdet", lambda: _kernels.slogdet(A)),
                         (f"xxl_{kind}_{n}_slogdet_parts", lambda: _kernels.slogdet_parts(A)),
                         (f"xxl_{kind}_{n}_slogpf", lambda: _kernels.slogpf(S, False)),
                         (f"xxl_{kind}_{n}_slogpf_parts", lambda: _kernels.slogpf_parts(S, False))]:
            ms, wall = _time_gpu(fn, steps, warmup)
            lu = name.endswith("slogdet") or name.endswith("slogdet_parts")
            flops = (2.0 / 3.0 if lu else 1.0 / 3.0) * n ** 3 * (4 if kind == "c128" else 1)
            if name.endswith("_parts"):
                flops += 2.0 * n ** 3 * (4 if kind == "c128" else 1)
            out[name] = dict(name=name, B=1, n=n, ms=ms, wall=wall, rate=1 / (ms * 1e-3), bytes=2 * esz * n * n,
                             flops=flops, sample=None)
        del A, S
        torch.cuda.empty_cache()
    return out


def main():
    args = _parse()
    if args.gpus != 1:
        print(
            json.dumps({"error": "fermix_amd benchmarks one GPU only (the hot path shards "
                        "trivially over the batch; no multi-GPU run is part of this build)",
                        "n_gpus": args.gpus}),
            flush=True,
        )
        sys.exit(2)
    only = set(args.only.split(",")) if args.only else {"c1", "c2", "c3", "c4"}
    # The CPU legs run first, before anything initialises the GPU, so that the worker
    # processes of the all-core leg fork from a process without GPU state.
    cpu = None
    lib = None
    if not args.no_cpu and ("c2" in only or "c1" in only):
        which = "slogpf" if "c2" in only else "slogdet"
        A = _inputs(4096, 128, 0)[:64]
        sample = A - np.swapaxes(A, 1, 2) if which == "slogpf" else A
        info = host_info()
        workers = min(16, info["affinity_cpus"] or info["os_cpu_count"] or 1)
        rate, reps, t, allc = cpu_baseline(sample, which, workers)
        cpu = {
            "value": round(rate, 2),
            "unit": "matrices/s",
            "cores": 1,
            "kind": "port",
            "sample": f"oracle {which}_generic (numpy restatement of the reference's generic "
            f"path), the first {sample.shape[0]} of the 4096 n=128 matrices x "
            f"{reps} reps in {t:.1f} s, one thread; value_all_cores: {workers} processes of one "
            f"thread each over slices of the same sample for about 8 s",
            "value_all_cores": round(allc, 2) if allc else None,
            "cores_all": workers,
            **info,
        }
        print(f"# cpu baseline ({which}): {rate:.1f} matrices/s one thread, "
              f"{allc or 0:.1f} with {workers} processes", file=sys.stderr, flush=True)
    if not args.no_cpu and "c1" in only:
        rates = cpu_library()
        t1, tn = sorted(rates)[0], sorted(rates)[-1]
        lib = {
            "value": round(rates[t1], 1),
            "unit": "matrices/s",
            "cores": t1,
            "kind": "library",
            "value_threads": {str(k): round(v, 1) for k, v in rates.items()},
            "sample": f"numpy.linalg.slogdet (LAPACK getrf) on the full C1 batch (B = 4096, n = 128), "
            f"{t1} and {tn} threads; compare workloads.c1",
        }
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}), flush=True)
        sys.exit(1)
    res = {}
    if "c2" in only:
        res["c2"] = bench_c2(args.steps, args.warmup)
        print(f"# c2 slogpf fwd: {res['c2']['ms']:.4f} ms/step", file=sys.stderr, flush=True)
        res["c2_noskew"] = bench_c2(args.steps, args.warmup, skew_symmetrize=False)
        print(f"# c2 slogpf fwd (skew_symmetrize=False): {res['c2_noskew']['ms']:.4f} ms/step",
              file=sys.stderr, flush=True)
    if "c1" in only:
        res["c1"] = bench_c1(args.steps, args.warmup)
        print(f"# c1 slogdet fwd: {res['c1']['ms']:.4f} ms/step", file=sys.stderr, flush=True)
    if "c3" in only:
        res["c3"] = bench_c3(max(10, args.steps), max(2, args.warmup // 2))
        print(f"# c3 slogdet fwd+grad (API default prec, bf16x3): {res['c3']['ms']:.4f} ms/step",
              file=sys.stderr, flush=True)
        res["c3_ieee"] = bench_c3(max(10, args.steps), max(2, args.warmup // 2), prec="ieee")
        print(f"# c3 slogdet fwd+grad (prec=ieee): {res['c3_ieee']['ms']:.4f} ms/step", file=sys.stderr,
              flush=True)
    if "c4" in only:
        res["c4"] = bench_c4(max(10, args.steps // 2), 2)
        print(f"# c4 slogpf fwd+grad (API defaults, bf16x3): {res['c4']['ms']:.4f} ms/step", file=sys.stderr,
              flush=True)
        res["c4_ieee"] = bench_c4(max(10, args.steps // 2), 2, prec="ieee")
        print(f"# c4 slogpf fwd+grad (prec=ieee): {res['c4_ieee']['ms']:.4f} ms/step", file=sys.stderr,
              flush=True)
    if "f64" in only:
        for k, r in bench_f64(args.steps, args.warmup).items():
            res[k] = r
            print(f"# {k}: {r['ms']:.4f} ms/step ({r['rate']:.4g} matrices/s)", file=sys.stderr,
                  flush=True)
    if "xxl" in only:
        for k, r in bench_xxl(max(2, args.steps // 10), 1).items():
            res[k] = r
            print(f"# {k}: {r['ms']:.2f} ms/step ({r['flops'] / (r['ms'] * 1e-3) / 1e12:.2f} TFLOP/s)",
                  file=sys.stderr, flush=True)
    if "blk" in only:
        for k, r in bench_blocked(max(3, args.steps // 4), max(1, args.warmup // 2)).items():
            res[k] = r
            print(f"# {k}: {r['ms']:.4f} ms/step ({r['rate']:.4g} matrices/s)", file=sys.stderr,
                  flush=True)
    if args.copy_probe:
        x = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device="cuda").fill_(1.0)
        for _ in range(3):
            y = x.clone()
        torch.cuda.synchronize()
        del x, y
    head = (res.get("c2") or res.get("c1") or res.get("c3") or res.get("c4")
            or res.get("f64_slogpf_fwd") or res.get("blk_f64_slogdet_parts")
            or res.get("xxl_f32_8192_slogdet"))
    achieved = head["bytes"] / (head["ms"] * 1e-3) / 1e9
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": _measured_traffic(head["name"]),
    }
    workloads = {
        k: {"workload": v["name"], "B": v["B"], "n": v["n"], "ms_per_step": round(v["ms"], 5),
            "matrices_per_s": round(v["rate"], 1),
            "hbm_frac": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            **({"alg_tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 2)} if "flops" in v else {})}
        for k, v in res.items()
    }
    line = {
        "metric": "fp32 slogdet/slogpf matrices/s at B=4096,n=128; fwd+grad matrices/s at n=512",
        "value": round(head["rate"], 1),
        "unit": "matrices/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if head["name"].startswith(("f64", "blk_f64")) else "f32",
        "data": "synthetic (numpy default_rng(0) N(0,1); jax.random absent)",
        "config": {"workload": f"{head['name']} B={head['B']} n={head['n']}", "B": head["B"],
                   "n": head["n"], "skew_symmetrize": True if head is res.get("c2") else None,
                   "baseline_config": "configs[1]" if head is res.get("c2") else "configs[0]"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_library": lib,
        "workloads": workloads,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
