#!/usr/bin/env python3
"""Benchmark: GPT-2 XL (1.5B) fp16-weight batch-1 greedy decode on one MI355X.

Workload (the configuration the headline metric is quoted on): GPT-2 XL
(48 layers, n_embd 1600, 25 heads, ffn 6400, vocab 50257), fp16 weights with
fp32 accumulation, synthetic random-init weights N(0, 0.02), a 512-token
random prompt, then greedy decoding to fill the 1024-position context.

One step = the workload's whole decode phase: 511 greedy decode forwards at
positions 512..1022, each selecting its token on the device and feeding it
to the next, replayed from the same prefilled KV cache every step.  The
timed region covers K steps; `value` is decode tokens per second over it.
Prefill throughput (prompt tokens / prefill time) is reported beside it.

roofline: the dominant kernel is the persistent decode-step kernel
g2k_step_f16_tail (one cooperative launch per token running all 48 layers, the
lm_head and the greedy pick); achieved = algorithmic bytes per launch / the
mean launch duration from HIP events on the library stream around the 511
launches, bytes per token from the formula
  w*(L*(3E^2 + E^2 + 2EF) + E*V) + kvb*2*L*E*T + 4*(13*L*E + 2E) + w*2E + kvb*2*L*E
(weights, K/V reads over T = pos+1 positions, biases and LayerNorm
parameters, embedding rows, K/V writes), against MI355X's 8 TB/s HBM peak.

cpu_baseline: the CPU oracle (a C restatement of the reference kernels with
their accumulation order) on the host's cores, decoding a fixed sample of
the same workload -- 100 greedy forwards at positions spread evenly over the
GPU run's positions (mean attended length the same as the GPU's), each over
the KV cache the GPU run wrote and with the GPU run's token for that
position -- with the CPU model and thread placement.

parity: the prompt is the one of the configuration's oracle fixture
(tests/golden/model/<config>.npz, written by the CPU oracle from the same
synthetic weights); after the timed region the timed decode ids are
compared with the fixture's greedy ids (the first from prefill, then one per
decode forward) and the bench line reports how many leading ids agree, and
where they part, the oracle's top-2 logit gap at that step.

traffic: HBM bytes per launch of that kernel from rocprofv3 counter runs
(FETCH_SIZE and WRITE_SIZE, one run each), each scaled by what the same
counter reads for a plain device copy of known size (`--copy-probe`); the
figures are read from profiles/<kernel>_<config>_traffic.json when it
exists and matches this workload, else traffic is null.

Other configurations of the workload list (each with its own prompt and
decode length: small fp32 64+255, medium fp32 128+511, large fp32 and
fp16-weight 256+511) run with --config; the headline is XL.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
                       [--config small|medium|large|large16|xl]
       python bench.py --copy-probe   (device copies of 1 GiB, for counter calibration)
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gpt2-opencl-1.1_amd"))

METRIC = "batch-1 decode tok/s + % HBM roofline (GPT-2 XL fp16); prefill tok/s"
SEED = 0x67707432
HBM_PEAK_GBS = 8000.0
# name: (preset, fp16 weights, prompt tokens); decode forwards fill the
# context to 1024 positions, except GPT-2 small (255 forwards)
CONFIGS = {"small": ("small", False, 64, 255), "medium": ("medium", False, 128, 511),
           "large": ("large", False, 256, 511), "large16": ("large", True, 256, 511),
           "xl": ("xl", True, 512, 511)}
CPU_SAMPLE_FORWARDS = 100
FIXTURES = os.path.join(ROOT, "tests", "golden", "model")


def step_bytes(cfg, w_bytes, kv_bytes, positions):
    """Algorithmic HBM bytes of decode forwards at the given positions."""
    L, E, F, V = cfg.n_layer, cfg.n_embd, cfg.ffn_dim, cfg.vocab_size
    fixed = w_bytes * (L * (3 * E * E + E * E + 2 * E * F) + E * V) + 4 * (13 * L * E + 2 * E) \
        + w_bytes * 2 * E + kv_bytes * 2 * L * E
    return sum(fixed + kv_bytes * 2 * L * E * (p + 1) for p in positions)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


COPY_BYTES = 1 << 30


def traffic_file(kernel, config):
    return os.path.join(ROOT, "profiles", f"{kernel}_{config}_traffic.json")


def copy_probe():
    """Five device-to-device copies of COPY_BYTES (torch's copy kernel): the
    known-size reference for calibrating the FETCH_SIZE / WRITE_SIZE
    counters."""
    import torch
    x = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    y = torch.empty_like(x)
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "copies": 5}), flush=True)


def measured_traffic(kernel, config, workload):
    """HBM bytes per launch from the committed counter summary, if it was
    taken on this kernel and workload."""
    try:
        with open(traffic_file(kernel, config)) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel or t.get("workload") != workload:
        return None
    return t.get("bytes_per_launch")


def cpu_description():
    """CPU model, logical CPUs this process may run on, and their list."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = list(range(os.cpu_count() or 1))
    return model, allowed


def fixture(config, P):
    """(prompt, greedy ids, top-2 logits) of the configuration's oracle
    fixture, or None when it is absent or was made for another prompt
    length."""
    path = os.path.join(FIXTURES, f"{config}.npz")
    try:
        with np.load(path, allow_pickle=False) as z:
            fx = {k: z[k] for k in ("prompt", "ids", "top2")}
    except (OSError, KeyError, ValueError):
        return None
    return fx if len(fx["prompt"]) == P else None


def parity_record(fx, config, first_tok, out):
    """How many of the timed run's greedy ids (the prefill token, then one
    per decode forward) agree with the oracle fixture's, leading ones."""
    got = np.concatenate([[first_tok], out]).astype(np.int64)
    ref = fx["ids"].astype(np.int64)
    n = min(len(got), len(ref))
    diff = np.flatnonzero(got[:n] != ref[:n])
    rec = {"ids_agree": int(diff[0]) if diff.size else n, "of": n,
           "fixture": f"tests/golden/model/{config}.npz",
           "counted": "the prefill token, then one id per timed decode forward"}
    if diff.size:
        k = int(diff[0])
        rec["parts_at"] = {"step": k, "oracle_top2_gap": float(fx["top2"][k, 0] - fx["top2"][k, 1])}
    return rec


def cpu_baseline(g2, m, cfg, f16, P, first_tok, out, n_forwards=CPU_SAMPLE_FORWARDS):
    """Time the oracle on a fixed sample of the same workload: n_forwards
    greedy decode forwards at positions spread evenly over the GPU run's
    decode positions P..P+len(out)-1, each over the KV cache the GPU run
    wrote, with the token the GPU run fed at that position (the reference's
    timing method, main.c:2106-2170: wall clock around the decode loop,
    sampling included, no printing).  The sample's mean attended length is
    the GPU run's."""
    sys.path.insert(0, ROOT)
    from oracle import oracle
    t0 = time.perf_counter()
    w = g2.synth_weights(cfg, SEED, f16_round=f16)
    om = oracle.Model(cfg, w, kslice=4)
    del w
    for l in range(cfg.n_layer):
        k, v = m.read_kv(l)
        om.set_kv(l, k, v)
    log(f"cpu oracle ready in {time.perf_counter() - t0:.1f}s")
    n_dec = len(out)
    toks = np.concatenate([[first_tok], out[:-1]]).astype(np.int64)  # token fed at position P + j
    n = min(n_forwards, n_dec)
    js = np.unique(np.linspace(0, n_dec - 1, n).round().astype(int))
    n = len(js)
    om.decode(int(toks[js[0]]), P + int(js[0]))  # untimed first forward (page-in)
    t0 = time.perf_counter()
    for j in js:
        om.decode(int(toks[j]), P + int(j))
        om.greedy([int(toks[j])], forbid_eos=True)
    dt = time.perf_counter() - t0
    mean_t = float(np.mean(P + js + 1))
    threads = oracle.num_threads()
    om.close()
    model, allowed = cpu_description()
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu": model, "logical_cpus_allowed": len(allowed),
            "pinning": (f"OpenMP threads {threads} (OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')}), "
                        f"no explicit binding; process affinity CPUs {allowed[0]}-{allowed[-1]}"
                        if allowed else "none"),
            "sample": f"{n} greedy decode forwards of GPT-2 {cfg.n_layer}-layer E{cfg.n_embd} "
                      f"({'fp16-rounded weights held as fp32' if f16 else 'fp32 weights'}) at positions spread "
                      f"evenly over {P}..{P + n_dec - 1} (mean attended length {mean_t:.0f}, as the GPU run's), "
                      f"over the GPU run's KV cache, {threads} OpenMP threads, {dt:.2f} s"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--config", default="xl", choices=list(CONFIGS),
                    help="xl: XL fp16 512+511 (default, the headline); small/medium/large: fp32 weights; "
                         "large16: large with fp16 weights")
    ap.add_argument("--copy-probe", action="store_true", help="device copies of 1 GiB for counter calibration")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe()
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this library runs on one GPU only; --gpus {args.gpus} (WORLD_SIZE {world}) is not "
              f"supported. Sharding the batch-1 decode by output columns across GPUs is designed but not "
              f"built; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import g2hip as g2
    g2.init(0)
    try:
        run(args, g2)
    finally:
        # release the model and the library before the interpreter exits, so
        # no HIP stream, module or buffer is left to the runtime's exit path
        g2.shutdown()


def run(args, g2):
    name, cus = g2.device_name()
    preset, f16, P, n_dec = CONFIGS[args.config]
    cfg = g2.preset(preset)
    wdtype = g2.F16 if f16 else g2.F32
    t0 = time.perf_counter()
    m = g2.Model.synth(cfg, SEED, wdtype, g2.PATH_FUSED)
    log(f"{args.config} model on {name} ({cus} CUs) in {time.perf_counter() - t0:.1f}s, "
        f"{m.weight_bytes() / 2**20:.0f} MiB of weights")
    fx = fixture(args.config, P)
    if fx is not None:
        prompt = fx["prompt"].astype(np.int32)
    else:
        log(f"no oracle fixture for {args.config}: random prompt, parity not reported")
        prompt = np.random.default_rng(SEED).integers(0, cfg.vocab_size, P).astype(np.int32)

    # prefill: prompt -> first token (device-selected), timed by HIP events
    ids, _ = m.generate(prompt, 2)  # warm-up, builds the decode graph
    prefill_ms = []
    for _ in range(3):
        ids, (pf_ms, _) = m.generate(prompt, 1)
        prefill_ms.append(pf_ms)
    first_tok = int(ids[0])
    prefill_tok_s = P / (min(prefill_ms) * 1e-3)

    # decode: W untimed steps, then K timed steps of 511 forwards each
    ref_ids = None
    for _ in range(args.warmup):
        ref_ids, _ = m.decode_run(first_tok, P, n_dec)
    g2.sync()
    ev_ms = []
    t_start = time.perf_counter()
    for _ in range(args.steps):
        out, ms = m.decode_run(first_tok, P, n_dec)
        ev_ms.append(ms)
        if ref_ids is None:
            ref_ids = out
        elif not np.array_equal(out, ref_ids):
            raise SystemExit("bench.py: decode steps disagree with each other (non-deterministic output)")
    g2.sync()
    wall = time.perf_counter() - t_start
    tok_s = args.steps * n_dec / wall
    step_ms_events = float(np.mean(ev_ms))
    bytes_step = step_bytes(cfg, 2 if f16 else 4, 4, range(P, P + n_dec))
    achieved = bytes_step / (step_ms_events * 1e-3) / 1e9

    kind = m.step_kind()
    kname = m.step_kernel() if kind else ""
    workload = (f"GPT-2 {preset.upper()} {'fp16' if f16 else 'fp32'}-weight batch-1 greedy decode: {P}-token "
                f"random prompt, {n_dec} decode forwards (positions {P}..{P + n_dec - 1})")
    result = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16" if f16 else "f32", "data": "synthetic",
        "config": {"workload": workload,
                   "weights": "f16" if f16 else "f32", "kv_cache": "f32", "accumulate": "f32",
                   "decode_engine": "persistent step kernel" if m.uses_step() else
                   ("per-operator kernels, graph replay" if m.uses_graph() == 1 else "per-operator kernels")},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "prefill_ms": round(min(prefill_ms), 3),
        "decode_ms_per_token": round(step_ms_events / n_dec, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(kname, args.config, workload) if kname else None,
                     "kernel": (f"{kname} (one launch per decode token)" if kname
                                else "decode step (per-operator kernels)"),
                     "bytes_per_launch": round(bytes_step / n_dec)},
    }
    result["parity"] = parity_record(fx, args.config, first_tok, ref_ids) if fx is not None else None
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(g2, m, cfg, f16, P, first_tok, ref_ids)
    print(json.dumps(result), flush=True)
    m.free()


if __name__ == "__main__":
    main()
