#!/usr/bin/env python3
"""DeltaAttention prefill benchmark on one MI355X.

Metric: prefill attention ms/layer and speedup over the dense flash
prefill, Llama-3-8B GQA shape (32 query heads, 8 KV heads, head_dim 128), bf16, causal.
A step is one layer's delta prefill attention: anchor selection -> index/pack/counts ->
two-phase hybrid prefill, on synthetic inputs already resident in HBM (the work the
reference times as time_get_row_delta + time_delta_mm_pattern,
modeling_llama.py:612-754).

The default run measures config 1 (N = 32768, r = 4) as the headline and adds to the same
JSON line: config 2 (N = 131072) at r = 2, 4 and 8, the same layer at N = 262144 and r = 4
(the reference's longest point, key ``n262144_r4``), config 0 in fp32 (``config0_fp32``),
the config-4 ragged batch, the config-3 end-to-end 32-layer prefill, the per-token decode
after the config-1 prefill (``decode``: the one-call step, and the decode attention against
the same kernels over the dense cache), the selection in both arithmetic definitions, the
on-box MFMA and copy ceilings, and the CPU baseline (config 1 and config 0 in full).
``--config 2`` runs N = 131072 alone with ``--ratio`` in {2, 4, 8}.  The threshold tau is
calibrated on the seeded keys so that the realised compression is r (smallest tau with
keep rate <= 1/r), in the selection arithmetic that is timed.

``--only {delta,hybrid,dense,compress}`` runs just that part for K steps (used for
rocprofv3 captures) and prints a short line instead of the JSON record.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    # the power manager settles within about 15 launches after idle or after a change of
    # load (the first launches run 5-25 % slow); 20 untimed steps let the timed ones start
    # in its steady state
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=(1, 2, 3, 4),
                    help="1: one layer at 32K; 2: one layer at 128K; 3: full 32-layer "
                         "Llama-3-8B prefill of 65536 tokens (tokens/s, attention share); "
                         "4: ragged batch of 8 sequences, 4096-32768 tokens each (varlen)")
    ap.add_argument("--e2e-mode", choices=("periodic", "delta"), default="periodic",
                    help="config 3 anchor selection: periodic with period r (the control "
                         "mapping; random-init keys are nearly independent, so delta keeps "
                         "almost everything) or delta with --tau")
    ap.add_argument("--tau", type=float, default=15.0)
    ap.add_argument("--e2e-layers", type=int, default=32)
    ap.add_argument("--ratio", type=float, default=4.0)
    ap.add_argument("--seq", type=int, default=0, help="override the sequence length")
    ap.add_argument("--window", type=int, default=128)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--dtype", choices=("bf16", "fp16"), default="bf16",
                    help="16-bit type of Q, K, V (configs 1 and 2); bf16 is the headline")
    ap.add_argument("--select-arith", choices=("native", "fp32"), default="native",
                    help="Euclidean distance of the anchor selection: the keys' own 16-bit "
                         "arithmetic as the reference computes it (tritonModules.py:55-58), or fp32")
    ap.add_argument("--only", choices=("delta", "hybrid", "dense", "compress", "copy", "convert", "peaks"),
                    default=None,
                    help="run one part for K steps (copy: a 1 GiB device copy; convert: 1 GiB of fp32 "
                         "read and written as bf16 by a vectorized elementwise kernel -- the "
                         "references for calibrating the WRITE_SIZE / FETCH_SIZE counters; peaks: "
                         "the on-box MFMA and copy ceilings, printed as JSON)")
    ap.add_argument("--decode", action="store_true",
                    help="per-token decode latency over the compressed cache left by a "
                         "config-1 prefill (update + attention), against the same decode "
                         "attention over the uncompressed cache")
    ap.add_argument("--decode-tokens", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-262k", action="store_true",
                    help="leave the N = 262144, r = 4 point out of the default run")
    ap.add_argument("--no-128k", action="store_true",
                    help="config 1 only: skip the config-2 (N=131072, r=2/4/8) measurements")
    ap.add_argument("--no-e2e", action="store_true",
                    help="config 1 only: skip the config-3 end-to-end, config-4 ragged-batch, config-0 "
                         "fp32 and decode parts")
    ap.add_argument("--no-sdpa", action="store_true",
                    help="skip timing torch's scaled_dot_product_attention as a second dense control")
    return ap.parse_args()


def parse_args_defaults():
    return {"steps": 30, "warmup": 5}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(q, k, v, tau, window, arith):
    """Time the reference's attention math on the GPU box's host cores, in full (no
    sampling or extrapolation): the CPU restatement of the delta step (selection by the
    C oracle in the same arithmetic as the GPU step, packing, then the hybrid attention)
    and of the dense eager attention (modeling_llama.py:235-276), both with torch's
    fused CPU attention (oracle/cpu_baseline.py), for config 1 (the given layer) and
    config 0 (B=1, 8 heads, head_dim 64, N=2048, fp32, r=4)."""
    import numpy as np
    import torch
    from oracle import cpu_baseline as CB
    from oracle import delta_oracle as O
    from oracle import select_oracle_c as OC
    from deltaattention_amd import synth

    cores = min(16, os.cpu_count() or 1)
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(cores)
    o_arith = "fp32" if arith == "fp32" else ("fp16" if k.dtype == torch.float16 else "bf16")

    def delta_and_dense(qc, kc, vc, tau_, W, sel_arith):
        kf, vf = kc.float().numpy(), vc.float().numpy()
        t0 = time.perf_counter()
        keep, _ = OC.select_delta(kf, tau_, 512, arith=sel_arith)
        p = O.pack(kf, vf, keep)
        t1 = time.perf_counter()
        CB.hybrid_attention(qc, kc, vc, p["k_packed"], p["v_packed"], p["timestamps"], p["counts"], W)
        t2 = time.perf_counter()
        CB.dense_attention(qc, kc, vc, True)
        t3 = time.perf_counter()
        return (t1 - t0), (t2 - t1), (t3 - t2), p["P"]

    try:
        qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
        t_comp, t_hyb, t_dense, P1 = delta_and_dense(qc, kc, vc, tau, window, o_arith)
        del qc, kc, vc
        # config 0: the CPU-runnable case of BASELINE.json, fp32, tau calibrated to r = 4 on
        # its keys by the oracle's selection
        q0, k0, v0 = synth.make_layer_inputs(1, 8, 8, 2048, 64, rope_base=10000.0, seed=0,
                                            dtype=torch.float32)
        k0f = k0.numpy()
        lo, hi = 0.0, 64.0
        for _ in range(30):
            mid = 0.5 * (lo + hi)
            if OC.select_delta(k0f, mid, 512)[1].sum() > k0f.shape[1] * k0f.shape[2] / 4.0:
                lo = mid
            else:
                hi = mid
        c0 = delta_and_dense(q0, k0, v0, hi, 128, "fp32")  # fp32 keys: fp32 arithmetic
    finally:
        torch.set_num_threads(prev_threads)
    return {"value": round(1e3 * (t_comp + t_hyb), 1), "unit": "ms/layer", "cores": cores, "kind": "port",
            "dense_value": round(1e3 * t_dense, 1),
            "select_pack_ms": round(1e3 * t_comp, 1), "hybrid_ms": round(1e3 * t_hyb, 1),
            "config0": {"delta_ms": round(1e3 * (c0[0] + c0[1]), 2), "dense_ms": round(1e3 * c0[2], 2),
                        "tau": round(hi, 4), "P": int(c0[3]),
                        "workload": "B=1 Hq=Hkv=8 D=64 N=2048 fp32 r=4, RoPE 1e4, fp32 selection"},
            "host_cpu_count": os.cpu_count(), "host_cpu": _cpu_model(),
            "sample": (f"config 1 in full, no extrapolation: the CPU restatement (oracle/) of the delta "
                       f"step -- C-oracle selection ({o_arith} arithmetic, as the GPU step) + numpy "
                       f"packing ({1e3 * t_comp:.0f} ms, P={P1}) + the hybrid attention over every "
                       f"query block through torch's fused CPU attention ({t_hyb:.1f} s) -- and the "
                       f"dense eager attention through the same ({t_dense:.1f} s); config 0 likewise "
                       f"(key 'config0'); torch threads={cores}")}


def traffic_bytes(args, N, r_real, ratio):
    """HBM bytes per launch of the hybrid attention kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (profiles/traffic_config*.json); None for a workload
    (sequence length, ratio, window, dtype) those runs do not cover."""
    if args.dtype != "bf16" or args.window != 128 or abs(r_real - ratio) > 0.05 * ratio:
        return None
    name = {32768: "traffic_config1.json", 131072: f"traffic_config2_r{int(ratio)}.json"}.get(N)
    if name is None:
        return None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            rec = json.load(f)
        if abs(float(rec.get("ratio", 4.0)) - ratio) > 1e-6:
            return None
        return int(rec["bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def config3_record(args, warmup, steps):
    """Config 3: 32-layer Llama-3-8B prefill of one 65536-token sequence, random bf16
    weights ~ N(0, 0.02), uniform token ids; PATH 1 (delta) and PATH 2 (dense) through
    the same model (modeling swap, llama_swap), ``warmup`` untimed and ``steps`` timed
    prefills per path.  Returns the record."""
    import torch
    from deltaattention_amd import globVR, llama_swap
    dev = torch.device("cuda:0")
    N = args.seq if args.config == 3 and args.seq else 65536
    cfg = llama_swap.llama3_8b_config(llama_swap.DELTA, num_layers=args.e2e_layers)
    log(f"config 3: {args.e2e_layers} layers, N={N}, building the model ...")
    t0 = time.perf_counter()
    model = llama_swap.random_llama(cfg, dev, seed=args.seed)
    g = torch.Generator().manual_seed(args.seed)
    ids = torch.randint(0, cfg.vocab_size, (1, N), generator=g).to(dev)
    torch.cuda.synchronize()
    log(f"model built in {time.perf_counter() - t0:.1f} s")
    saved = dict(vars(globVR))
    res = {}
    try:
        if args.e2e_mode == "periodic":
            globVR.packing_mode = "periodic"
            globVR.target_keep_rate = 1.0 / args.ratio
        else:
            globVR.packing_mode = "delta"
            globVR.row_delta_threshold = args.tau
            globVR.chunk_size = 512
        globVR.row_delta_arith = args.select_arith
        globVR.dense_window_size = args.window
        for name in (llama_swap.DELTA, llama_swap.DENSE):
            llama_swap.set_implementation(model, name)
            with torch.no_grad():
                for _ in range(warmup):
                    model(ids, use_cache=False)
                torch.cuda.synchronize()
                times, att = [], []
                for _ in range(steps):
                    llama_swap.reset_attention_time()
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    model(ids, use_cache=False)
                    torch.cuda.synchronize()
                    times.append(time.perf_counter() - t0)
                    att.append(llama_swap.attention_time_ms())
            ms = 1e3 * sum(times) / len(times)
            res[name] = (ms, sum(att) / len(att))
            log(f"{name}: {ms:.1f} ms per prefill, attention {res[name][1]:.1f} ms")
    finally:
        for name, val in saved.items():
            setattr(globVR, name, val)
        del model
        torch.cuda.empty_cache()
    ms_delta, att_delta = res[llama_swap.DELTA]
    ms_dense, att_dense = res[llama_swap.DENSE]
    return {
        "metric": "prefill tokens/s, full Llama-3-8B (32 layers), delta attention",
        "value": round(N / (ms_delta * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_delta, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": (f"synthetic: random bf16 weights N(0,0.02), {N} uniform token ids, seed "
                 f"{args.seed}; anchors {args.e2e_mode} "
                 + (f"period {args.ratio:g}" if args.e2e_mode == "periodic" else f"tau {args.tau:g}")
                 + f", W={args.window}; logits over all positions"),
        "config": {"workload": f"config3: {args.e2e_layers}-layer Llama-3-8B prefill, N={N}",
                   "seq_len": N, "global_batch": 1, "parallelism": "none (1 GPU)"},
        "attention_share_delta": round(att_delta / ms_delta, 4),
        "attention_ms_delta": round(att_delta, 2),
        "dense_tokens_per_s": round(N / (ms_dense * 1e-3), 1),
        "dense_ms_per_step": round(ms_dense, 2),
        "attention_share_dense": round(att_dense / ms_dense, 4),
        "attention_ms_dense": round(att_dense, 2),
        "speedup_vs_dense": round(ms_dense / ms_delta, 3),
        "attention_speedup_vs_dense": round(att_dense / att_delta, 3),
    }


def run_config3(args):
    print(json.dumps(config3_record(args, args.warmup, args.steps)), flush=True)


def run_decode(args):
    print(json.dumps(decode_record(args)), flush=True)


def decode_record(args):
    """Per-token decode (deltaDecoding.py:181-362 as modeling_llama.py:453-518 drives it)
    after a config-1 prefill: the compressed cache holds the P packed anchors of the
    delta selection plus the last W keys in the ring; each token runs the cache update
    and the decode attention for one layer.  The control is the same decode attention
    over an uncompressed cache (all N keys packed with count 1, empty ring).  Returns the
    record (bench.py --decode prints it as its JSON line)."""
    import types
    import torch
    from deltaattention_amd import deltaDecoding as dd
    from deltaattention_amd import globVR, ops, synth
    dev = torch.device("cuda:0")
    N = args.seq or 32768
    B, Hq, Hkv, D, W = 1, 32, 8, 128, args.window
    q, k, v = synth.make_layer_inputs(B, Hq, Hkv, N, D, rope_base=500000.0, seed=args.seed,
                                      device=dev, qv_on_device=True)
    tau, r_real = synth.calibrate_threshold(k, args.ratio, arith=args.select_arith)
    globVR.row_similarity_metric = "euclidean"
    globVR.row_delta_threshold = tau
    globVR.row_delta_arith = args.select_arith
    keep, _ = ops.select(k, tau, 512, arith=args.select_arith)
    packed = ops.pack(keep, k, v).trimmed()
    P = packed.k_packed.shape[2]
    cfg = types.SimpleNamespace(head_dim=D, num_key_value_heads=Hkv, num_hidden_layers=1,
                                hidden_size=Hq * D, num_attention_heads=Hq)
    T = args.decode_tokens
    gen = torch.Generator(device=dev).manual_seed(args.seed + 7)
    new_k = torch.randn((T, B, Hkv, 1, D), generator=gen, device=dev).to(torch.bfloat16)
    new_v = torch.randn((T, B, Hkv, 1, D), generator=gen, device=dev).to(torch.bfloat16)
    q_tok = torch.randn((T, B, Hq, 1, D), generator=gen, device=dev).to(torch.bfloat16)

    def compressed_cache():
        c = dd.HybridCompressedCache(cfg, B, dtype=torch.bfloat16, exact_window_size=W,
                                     initial_capacity=P + T + 1024, device=dev)
        c.initialize_from_prefill(0, packed.k_packed, packed.v_packed, packed.counts,
                                  packed.timestamps, k[:, :, N - W:], v[:, :, N - W:], N)
        return c

    dense = dd.HybridCompressedCache(cfg, B, dtype=torch.bfloat16, exact_window_size=W,
                                     initial_capacity=N + 1024, device=dev)
    dense.initialize_from_prefill(0, k, v, torch.ones((B, Hkv, N), dtype=torch.int32, device=dev),
                                  torch.arange(N, dtype=torch.int32, device=dev).expand(B, Hkv, N),
                                  k[:, :, :0], v[:, :, :0], N)

    def timed(fn, n):
        st = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(st)
        for i in range(n):
            fn(i)
        e1.record(st)
        e1.synchronize()
        return e0.elapsed_time(e1) / n

    for _ in range(2):  # warm-up on throw-away caches
        c = compressed_cache()
        c2 = compressed_cache()
        for i in range(8):
            c.update(new_k[i], new_v[i], 0)
            dd.decode_attention(q_tok[i], c, 0)
            dd.decode_attention(q_tok[i], dense, 0)
            c2.decode_step(q_tok[i], new_k[i], new_v[i], 0)
    cache = compressed_cache()
    fused = compressed_cache()
    last = {}

    def step(i):
        cache.update(new_k[i], new_v[i], 0)
        last["two"] = dd.decode_attention(q_tok[i], cache, 0)

    def fused_step(i):
        last["one"] = fused.decode_step(q_tok[i], new_k[i], new_v[i], 0)

    ms_two = timed(step, T)
    ms_delta = timed(fused_step, T)
    # the one-call step leaves the same cache as the two calls, and the same last output up
    # to rounding (its key list holds the evicted token after the ring, not before it)
    step_err = float((last["one"].float() - last["two"].float()).abs().max())
    if not (step_err <= 1e-2
            and torch.equal(fused.packed_lengths, cache.packed_lengths)
            and torch.equal(fused.packed_counts, cache.packed_counts)
            and torch.equal(fused.k_packed, cache.k_packed)
            and torch.equal(fused.v_packed, cache.v_packed)
            and torch.equal(fused.k_exact, cache.k_exact)):
        raise RuntimeError(f"decode_step differs from update + decode_attention (max-abs {step_err:.3e})")
    ms_attn = timed(lambda i: dd.decode_attention(q_tok[i], cache, 0), T)
    ms_dense = timed(lambda i: dd.decode_attention(q_tok[i], dense, 0), T)

    # GPU time of the decode attention without the host launch path: 32 calls (one per
    # layer of a decode step) captured in one HIP graph and replayed, so the kernels run
    # back to back; every replay is checked against the eager result
    LAYERS = 32

    def graph_ms(c):
        qg = q_tok[0].clone()
        ref = dd.decode_attention(qg, c, 0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs_g = [dd.decode_attention(qg, c, 0) for _ in range(LAYERS)]
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            if not all(torch.equal(o, ref) for o in outs_g):
                raise RuntimeError("decode attention graph replay differs from the eager call")
        return timed(lambda i: g.replay(), max(1, T // LAYERS)) / LAYERS

    gms_delta = graph_ms(cache)
    gms_dense = graph_ms(dense)
    log(f"decode: delta {ms_delta * 1e3:.1f} us/token in one call ({ms_two * 1e3:.1f} as update + "
        f"attention; attention {ms_attn * 1e3:.1f}, graph "
        f"{gms_delta * 1e3:.1f}), dense attention {ms_dense * 1e3:.1f} (graph "
        f"{gms_dense * 1e3:.1f}) us/token, P={P}")
    rec = {
        "metric": "decode us/token/layer, compressed cache vs dense, Llama-3-8B GQA",
        "value": round(ms_delta * 1e3, 2), "unit": "us/token/layer",
        "n_gpus": 1, "steps": T, "warmup": 16, "ms_per_step": round(ms_delta, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": (f"synthetic: config-1 prefill (AR(1) keys, seed {args.seed}, tau={tau:.4f}, "
                 f"realised r={r_real:.3f}) then {T} random decode tokens"),
        "config": {"workload": f"decode after an N={N} prefill: B=1 Hq=32 Hkv=8 D=128, "
                               f"P={P} anchors + W={W} ring",
                   "seq_len": N, "global_batch": B, "parallelism": "none (1 GPU)"},
        "two_call_us_delta": round(ms_two * 1e3, 2),
        "attention_us_delta": round(ms_attn * 1e3, 2),
        "update_us_delta": round((ms_two - ms_attn) * 1e3, 2),
        "attention_us_dense": round(ms_dense * 1e3, 2),
        "attention_gpu_us_delta": round(gms_delta * 1e3, 2),
        "attention_gpu_us_dense": round(gms_dense * 1e3, 2),
        "attention_gpu_speedup_vs_dense": round(gms_dense / gms_delta, 3),
        "note": ("value is HybridCompressedCache.decode_step (update + attention in one "
                 "da_decode_step call), two_call_us_delta the same token as cache.update + "
                 "decode_attention; value and the *_us fields are host-inclusive (Python + "
                 "launch per call); the *_gpu_us fields replay 32 decode attentions captured "
                 "in one graph, per call"),
        "keys_delta": P + W, "keys_dense": N,
    }
    return rec


def config4_record(args, warmup, steps):
    """Config 4: a packed ragged batch of 8 sequences with N_b ~ U[4096, 32768] tokens,
    AR(1) keys with rho ~ U[0.6, 0.95] per (sequence, KV head), one tau calibrated to r
    on the whole batch.  ops.delta_prefill_varlen runs every sequence as a B = 1 delta
    prefill with one launch per stage over the whole batch (cu_seqlens on the device),
    against the dense varlen prefill (one launch).  Returns the record."""
    import numpy as np
    import torch
    from deltaattention_amd import ops, synth
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(args.seed)
    lens = rng.integers(4096, 32768, size=8, endpoint=True).tolist()
    Hq, Hkv, D = 32, 8, 128
    qs, ks, vs = [], [], []
    for i, n in enumerate(lens):
        rho = rng.uniform(0.6, 0.95, size=Hkv)
        q, k, v = synth.make_layer_inputs(1, Hq, Hkv, n, D, rho=rho, rope_base=500000.0,
                                          seed=args.seed * 100 + i, device=dev, qv_on_device=True)
        qs.append(q[0].permute(1, 0, 2))
        ks.append(k[0].permute(1, 0, 2))
        vs.append(v[0].permute(1, 0, 2))
    q, k, v = torch.cat(qs).contiguous(), torch.cat(ks).contiguous(), torch.cat(vs).contiguous()
    del qs, ks, vs
    cu = [0] + np.cumsum(lens).tolist()
    T = cu[-1]
    log(f"config 4: lens {lens}, {T} tokens")
    tau, _ = synth.calibrate_threshold(k.permute(1, 0, 2).unsqueeze(0), args.ratio, arith=args.select_arith)
    vb = ops.varlen_batch(cu, T, dev)
    keep, _ = ops.select_varlen(k, vb, tau, 512, arith=args.select_arith)
    r_real = T * Hkv / int(keep.sum().item())

    def delta():
        return ops.delta_prefill_varlen(q, k, v, vb, tau, 512, window=args.window, arith=args.select_arith)

    def dense():
        return ops.dense_prefill_varlen(q, k, v, vb)

    res = {}
    for name, fn in (("delta", delta), ("dense", dense)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        res[name] = 1e3 * (time.perf_counter() - t0) / steps
        log(f"{name}: {res[name]:.2f} ms per batch")
    return {
        "metric": "ragged-batch prefill attention tokens/s (8 sequences, varlen), delta",
        "value": round(T / (res["delta"] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(res["delta"], 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": (f"synthetic: AR(1) keys with rho~U[0.6,0.95] per sequence and KV head, RoPE "
                 f"base 5e5, Gaussian Q/V, seed {args.seed}; Euclidean tau={tau:.4f} calibrated "
                 f"to r={args.ratio:g} on the batch (realised {r_real:.3f}, {args.select_arith} "
                 f"selection), chunk 512, W={args.window}"),
        "config": {"workload": f"config4: varlen B=8 lens {lens}, Hq={Hq} Hkv={Hkv} D={D} bf16 causal",
                   "seq_len": T, "global_batch": 8, "parallelism": "none (1 GPU)"},
        "delta_ms_per_batch": round(res["delta"], 3),
        "dense_tokens_per_s": round(T / (res["dense"] * 1e-3), 1),
        "dense_ms_per_batch": round(res["dense"], 3),
        "speedup_vs_dense": round(res["dense"] / res["delta"], 3),
        "realised_ratio": round(r_real, 3),
    }


def run_config4(args):
    print(json.dumps(config4_record(args, args.warmup, args.steps)), flush=True)


def config0_record(args):
    """Config 0 as BASELINE.json states it, on the GPU: B=1, 8 query and 8 KV heads,
    head_dim 64, N=2048, fp32 tensors (fp32 selection, packing and attention), RoPE base
    1e4, tau calibrated to r = 4 by the GPU selection; the same inputs as the CPU
    baseline's config-0 leg.  HIP-event time of the whole delta step and of the dense
    prefill, 20 warm-up and 50 timed calls each."""
    import torch
    from deltaattention_amd import ops, synth
    dev = torch.device("cuda:0")
    q, k, v = (t.to(dev) for t in synth.make_layer_inputs(1, 8, 8, 2048, 64, rope_base=10000.0, seed=0,
                                                           dtype=torch.float32))
    tau, r_real = synth.calibrate_threshold(k, 4.0)
    step = lambda: ops.delta_prefill(q, k, v, tau, 512, window=args.window)
    dense = lambda: ops.dense_prefill(q, k, v)
    for _ in range(20):
        step(), dense()
    ms_step, ms_dense = time_loop(step, 50), time_loop(dense, 50)
    log(f"config 0 (fp32): delta {ms_step:.3f} ms, dense {ms_dense:.3f} ms")
    return {"delta_ms": round(ms_step, 4), "dense_ms": round(ms_dense, 4),
            "speedup_vs_dense": round(ms_dense / ms_step, 3), "tau": round(tau, 4),
            "realised_ratio": round(r_real, 3),
            "workload": "config0: B=1 Hq=Hkv=8 D=64 N=2048 fp32 r=4, RoPE 1e4 (fp32 selection and attention)"}


def measure_peaks():
    """On-box ceilings for the roofline fractions, each the best of 5 timed launches after a
    warm-up:

    * the bf16 MFMA rate of an issue loop with no memory traffic (libdeltaattn_diag.so:
      1024 workgroups x 8 waves x 32 MFMAs per round), once with constant operands and once
      with random N(0, 1) operands, with the shader clock each holds (s_memtime cycles over
      s_memrealtime's 100 MHz).  The chip's power limit lowers the clock as the multiplier
      arrays switch: only the constant-operand loop comes near the published peak, and the
      random-operand loop is the ceiling that data-bearing MFMA work (attention) can reach;
    * the HBM bandwidth of a 4 GiB device-to-device copy (bytes read + written)."""
    import torch
    here = os.path.dirname(os.path.abspath(__file__))
    lib = ctypes.CDLL(os.path.join(here, "deltaattention_amd", "libdeltaattn_diag.so"))
    lib.diag_mfma_loop.restype = ctypes.c_int
    lib.diag_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_void_p]
    lib.diag_mfma_operand_count.restype = ctypes.c_int64
    grid, iters = 1024, 4000
    sink = torch.empty(grid * 512, dtype=torch.float32, device="cuda")
    clocks = torch.zeros(grid * 4, dtype=torch.int64, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(1)
    operands = torch.randn(lib.diag_mfma_operand_count() * 8, dtype=torch.float32, device="cuda",
                           generator=gen).to(torch.bfloat16)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    flops = grid * 8 * iters * 32 * 32768.0

    def loop(ops):
        def run():
            rc = lib.diag_mfma_loop(ctypes.c_void_p(sink.data_ptr()), ops, ctypes.c_void_p(clocks.data_ptr()),
                                    iters, grid, stream)
            if rc != 0:
                raise RuntimeError(f"diag_mfma_loop failed ({rc})")
        run()
        best = min(time_loop(run, 1) for _ in range(5))
        c = clocks.view(grid, 4).cpu().double()
        ghz = ((c[:, 1] - c[:, 0]) / ((c[:, 3] - c[:, 2]) * 10.0)).median().item()
        return flops / (best * 1e-3) / 1e12, ghz

    const_tf, const_ghz = loop(None)
    live_tf, live_ghz = loop(ctypes.c_void_p(operands.data_ptr()))
    n = 1 << 31  # 2^31 bf16 elements: 4 GiB
    src = torch.empty(n, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    copy = lambda: dst.copy_(src)
    copy()
    best_copy = min(time_loop(copy, 1) for _ in range(5))
    del src, dst, sink, operands, clocks
    torch.cuda.empty_cache()
    copy_gbs = 2.0 * n * 2 / (best_copy * 1e-3) / 1e9
    log(f"peaks: MFMA loop {const_tf:.0f} TFLOP/s at {const_ghz:.2f} GHz (constant operands), "
        f"{live_tf:.0f} TFLOP/s at {live_ghz:.2f} GHz (random operands), copy {copy_gbs:.0f} GB/s")
    return {"mfma_bf16_tflops": round(const_tf, 1), "mfma_frac_of_published": round(const_tf / BF16_PEAK_TFLOPS, 4),
            "mfma_clock_ghz": round(const_ghz, 3),
            "mfma_live_bf16_tflops": round(live_tf, 1),
            "mfma_live_frac_of_published": round(live_tf / BF16_PEAK_TFLOPS, 4),
            "mfma_live_clock_ghz": round(live_ghz, 3),
            "copy_gbs": round(copy_gbs, 1), "copy_frac_of_published": round(copy_gbs / HBM_PEAK_GBS, 4),
            "note": "MFMA: v_mfma_f32_32x32x16_bf16 issue loop, no memory traffic, constant operands "
                    "(mfma_*) and random N(0,1) operands (mfma_live_*: the power limit lowers the "
                    "shader clock); copy: 4 GiB device-to-device, read + write bytes"}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; multi-GPU runs are not "
                                   "part of it (the path would shard by KV head: each GPU owns whole KV heads and "
                                   "their query heads, so attention needs no collective)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.config == 3:
        if args.steps == parse_args_defaults()["steps"]:
            args.steps = 2
        if args.warmup == parse_args_defaults()["warmup"]:
            args.warmup = 1
        run_config3(args)
        return
    if args.config == 4:
        run_config4(args)
        return
    if args.decode:
        run_decode(args)
        return
    if args.only == "peaks":
        print(json.dumps(measure_peaks()), flush=True)
        return
    if args.only:
        run_only(args)
        return
    import torch
    t_start = time.perf_counter()
    N = args.seq or (32768 if args.config == 1 else 131072)
    head = measure_layer(args, N, args.ratio, headline=True)
    rec = head.pop("record")
    cpu_inputs = head.pop("cpu_inputs")
    torch.cuda.empty_cache()
    full = args.config == 1 and not args.seq
    if full and not args.no_128k:
        # config 2: one set of N = 131072 inputs, tau calibrated per ratio; the dense and
        # SDPA controls do not depend on r and are timed once
        q, k, v = layer_inputs(args, 131072)
        shared = {}
        for r in (4.0, 2.0, 8.0):
            log(f"config 2 (N=131072, r={r:g}) ...")
            extra = measure_layer(args, 131072, r, headline=False, inputs=(q, k, v), shared=shared)
            rec[f"config2_r{int(r)}"] = extra
        del q, k, v, shared
        torch.cuda.empty_cache()
    if full and not args.no_262k:
        # the reference's longest point (eval_speedup.py:28): the config-2 layer at 262144
        # tokens, r = 4, with its own dense and SDPA controls
        log("N=262144, r=4 ...")
        q, k, v = layer_inputs(args, 262144)
        rec["n262144_r4"] = measure_layer(args, 262144, 4.0, headline=False, inputs=(q, k, v), shared={})
        del q, k, v
        torch.cuda.empty_cache()
    if full and not args.no_e2e:
        c4 = config4_record(args, warmup=20, steps=10)
        rec["config4"] = {key: c4[key] for key in (
            "delta_ms_per_batch", "dense_ms_per_batch", "speedup_vs_dense", "value", "unit",
            "dense_tokens_per_s", "realised_ratio", "steps", "warmup")}
        rec["config4"]["workload"] = c4["config"]["workload"]
        torch.cuda.empty_cache()
        c3 = config3_record(args, warmup=1, steps=1)
        rec["config3"] = {key: c3[key] for key in (
            "value", "unit", "ms_per_step", "dense_tokens_per_s", "dense_ms_per_step", "speedup_vs_dense",
            "attention_ms_delta", "attention_share_delta", "attention_ms_dense", "attention_share_dense",
            "attention_speedup_vs_dense", "steps", "warmup")}
        rec["config3"]["workload"] = c3["config"]["workload"] + f", anchors {args.e2e_mode} r={args.ratio:g}"
        torch.cuda.empty_cache()
        rec["config0_fp32"] = config0_record(args)
        torch.cuda.empty_cache()
        log("decode after the config-1 prefill ...")
        d = decode_record(args)
        rec["decode"] = {key: d[key] for key in (
            "value", "unit", "two_call_us_delta", "attention_us_delta", "attention_gpu_us_delta",
            "attention_gpu_us_dense", "attention_gpu_speedup_vs_dense", "keys_delta", "keys_dense", "steps")}
        rec["decode"]["metric"] = d["metric"]
        rec["decode"]["workload"] = d["config"]["workload"]
        torch.cuda.empty_cache()
    if full:
        rec["peaks_measured"] = measure_peaks()
        pk = rec["peaks_measured"]
        rec["roofline"]["frac_of_measured_peak"] = round(rec["roofline"]["achieved"] / pk["mfma_bf16_tflops"], 4)
        rec["roofline"]["frac_of_live_mfma_peak"] = round(rec["roofline"]["achieved"] / pk["mfma_live_bf16_tflops"], 4)
        rec["compress_frac_of_measured_copy"] = round(rec["compress_gbs"] / pk["copy_gbs"], 4)
    if not args.no_cpu_baseline:
        log("cpu baseline (config 1 and config 0 in full) ...")
        rec["cpu_baseline"] = cpu_baseline(*cpu_inputs, args.window, args.select_arith)
    rec["bench_wall_s"] = round(time.perf_counter() - t_start, 1)
    print(json.dumps(rec), flush=True)


def layer_inputs(args, N):
    import torch
    from deltaattention_amd import synth
    dev = torch.device("cuda:0")
    q, k, v = synth.make_layer_inputs(1, 32, 8, N, 128, rope_base=500000.0, seed=args.seed,
                                      device=dev, qv_on_device=True,
                                      dtype=torch.float16 if args.dtype == "fp16" else torch.bfloat16)
    torch.cuda.synchronize()
    return q, k, v


def time_loop(fn, iters):
    """Average ms per call of ``fn``, with HIP events on the stream the kernels run on."""
    import torch
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(st)
    for _ in range(iters):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


def cold_calls_ms(fn, runs=10, warm=3, flush_bytes=512 << 20):
    """Median and mean ms of ``fn`` over ``runs`` calls after ``warm`` untimed ones, each
    call preceded by writing a ``flush_bytes`` buffer (more than the 256 MB Infinity Cache
    plus the L2s), so that every call reads its inputs from HBM.  HIP events bracket each
    call on the stream the kernels run on."""
    import statistics
    import torch
    st = torch.cuda.current_stream()
    flush = torch.empty(flush_bytes, dtype=torch.uint8, device="cuda")
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    times = []
    for i in range(warm + runs):
        flush.fill_(i & 0xFF)
        e0.record(st)
        fn()
        e1.record(st)
        e1.synchronize()
        if i >= warm:
            times.append(e0.elapsed_time(e1))
    del flush
    return statistics.median(times), statistics.fmean(times)


def sdpa_ms(q, k, v, iters):
    """torch's scaled_dot_product_attention (causal) on the same inputs, flash / memory-
    efficient backends only (the math backend would materialise N x N), K/V expanded to
    the query heads; None when no such backend runs these shapes."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel
    G = q.shape[1] // k.shape[1]
    ke = k.repeat_interleave(G, dim=1).contiguous()
    ve = v.repeat_interleave(G, dim=1).contiguous()
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            fn = lambda: torch.nn.functional.scaled_dot_product_attention(q, ke, ve, is_causal=True)
            fn()
            torch.cuda.synchronize()
            return time_loop(fn, iters)
    except RuntimeError as e:
        log(f"sdpa unavailable: {e}")
        return None
    finally:
        del ke, ve


def measure_layer(args, N, ratio, headline, inputs=None, shared=None):
    """One Llama-3-8B attention layer (B=1, Hq=32, Hkv=8, D=128) at N tokens and
    compression r: the contract's timed steps of the full delta step (select -> pack ->
    hybrid) when ``headline``, then per-part HIP-event timings of the hybrid, dense,
    compression, selection and torch SDPA launches and the roofline of the hybrid
    kernel.  ``shared`` carries the r-independent dense / SDPA timings between calls at
    the same N.  Returns a dict; with ``headline``, ``record`` holds the JSON line's
    fields and ``cpu_inputs`` the layer for the CPU baseline."""
    import torch
    from deltaattention_amd import metrics, ops, synth
    W = args.window
    arith = args.select_arith
    other = "fp32" if arith == "native" else "native"
    B, Hq, Hkv, D = 1, 32, 8, 128
    log(f"layer: N={N} r={ratio} W={W} select={arith}")
    q, k, v = inputs if inputs is not None else layer_inputs(args, N)
    tau, r_real = synth.calibrate_threshold(k, ratio, arith=arith)
    log(f"calibrated tau={tau:.4f} realised r={r_real:.3f}")

    def step():
        return ops.delta_prefill(q, k, v, tau, 512, window=W, arith=arith)

    keep, _ = ops.select(k, tau, 512, arith=arith)
    packed = ops.pack(keep, k, v)
    torch.cuda.synchronize()
    P = int(packed.num_packed.item())
    ts_h = packed.timestamps[:, :, :P].cpu().numpy()
    c_h = packed.anchor_counts.cpu().numpy()
    out_h = torch.empty_like(q)
    out_d = torch.empty_like(q)

    def hybrid_only():
        ops.hybrid_prefill(q, k, v, packed.k_packed, packed.v_packed, packed.timestamps,
                           packed.counts, window=W, num_packed_dev=packed.num_packed, out=out_h)

    def dense_only():
        ops.dense_prefill(q, k, v, causal=True, out=out_d)

    def compress_only():
        kk, _ = ops.select(k, tau, 512, arith=arith)
        ops.pack(kk, k, v, out=packed)

    steps = args.steps if headline else max(3, min(args.steps, 10))
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms_step = 1e3 * (time.perf_counter() - t0) / steps
    log(f"delta step {ms_step:.3f} ms")

    iters = max(3, steps)
    shared = {} if shared is None else shared
    for _ in range(2):
        hybrid_only(); compress_only()
    ms_hybrid = time_loop(hybrid_only, iters)
    if "dense_ms" not in shared:
        dense_only()
        shared["dense_ms"] = time_loop(dense_only, iters)
        shared["sdpa_ms"] = sdpa_ms(q, k, v, max(3, iters // 3)) if not args.no_sdpa else None
    ms_dense, ms_sdpa = shared["dense_ms"], shared["sdpa_ms"]
    ms_compress = time_loop(compress_only, iters)
    cold_med, cold_mean = cold_calls_ms(compress_only)
    # the selection kernel alone, in the timed arithmetic and in the other definition (its
    # own tau, calibrated to the same r)
    tau_o, _ = synth.calibrate_threshold(k, ratio, arith=other)
    sel = {arith: time_loop(lambda: ops.select(k, tau, 512, arith=arith), iters),
           other: time_loop(lambda: ops.select(k, tau_o, 512, arith=other), iters)}
    log(f"hybrid {ms_hybrid:.3f} ms  dense {ms_dense:.3f} ms  compress {ms_compress:.4f} ms "
        f"(caches flushed: median {cold_med:.4f}, mean {cold_mean:.4f})  select native "
        f"{1e3 * sel['native']:.1f} us fp32 {1e3 * sel['fp32']:.1f} us  "
        f"sdpa {ms_sdpa if ms_sdpa is None else round(ms_sdpa, 3)} ms")

    fl = metrics.hybrid_flops(ts_h, c_h, P, N, Hq, D, W)
    dense_fl = metrics.dense_flops(B, Hq, N, D)
    cbytes = metrics.compression_bytes(N, D, c_h)
    hyb_tflops = fl["algorithmic"] / (ms_hybrid * 1e-3) / 1e12
    dense_tflops = dense_fl / (ms_dense * 1e-3) / 1e12
    best_dense = min(ms_dense, ms_sdpa) if ms_sdpa else ms_dense
    res = {
        "seq_len": N, "ratio": ratio, "realised_ratio": round(r_real, 3), "tau": round(tau, 4),
        "select_arith": arith,
        "delta_ms_per_layer": round(ms_step, 4),
        "speedup_vs_dense": round(ms_dense / ms_step, 3),
        "kernel_speedup_vs_dense": round(ms_dense / ms_hybrid, 3),
        "dense_ms_per_layer": round(ms_dense, 4),
        "sdpa_ms_per_layer": None if ms_sdpa is None else round(ms_sdpa, 4),
        "speedup_vs_best_dense": round(best_dense / ms_step, 3),
        "hybrid_kernel_ms": round(ms_hybrid, 4),
        "hybrid_algorithmic_flops": fl["algorithmic"],
        "compress_ms": round(ms_compress, 4),
        "compress_gbs": round(cbytes / (ms_compress * 1e-3) / 1e9, 1),
        "compress_hbm_frac": round(cbytes / (ms_compress * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "compress_cold_ms_median": round(cold_med, 4),
        "compress_cold_ms_mean": round(cold_mean, 4),
        "compress_cold_gbs": round(cbytes / (cold_med * 1e-3) / 1e9, 1),
        "select_native_us": round(1e3 * sel["native"], 2),
        "select_fp32_us": round(1e3 * sel["fp32"], 2),
        "hybrid_tflops": round(hyb_tflops, 1),
        "hybrid_mfma_frac": round(hyb_tflops / BF16_PEAK_TFLOPS, 4),
        # hardware utilisation at the reference's granularity: 4 D 128 128 per processed
        # (query block, key block) pair of its schedule; the kernel itself skips work at
        # 32-key x 64-row granularity, so its MFMA counters read less than this
        "hybrid_executed_tile_flops": fl["executed_tiles"],
        "hybrid_tile_tflops": round(fl["executed_tiles"] / (ms_hybrid * 1e-3) / 1e12, 1),
        "dense_tflops": round(dense_tflops, 1),
        "dense_mfma_frac": round(dense_tflops / BF16_PEAK_TFLOPS, 4),
    }
    if not headline:
        res["traffic"] = traffic_bytes(args, N, r_real, ratio)
        return res
    # the whole step in the other selection definition, for comparison
    for _ in range(3):
        ops.delta_prefill(q, k, v, tau_o, 512, window=W, arith=other)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ops.delta_prefill(q, k, v, tau_o, 512, window=W, arith=other)
    torch.cuda.synchronize()
    res[f"delta_ms_per_layer_{other}"] = round(1e3 * (time.perf_counter() - t0) / steps, 4)
    rec = {
        "metric": "prefill attn ms/layer + speedup vs dense FA at 32K/128K, Llama-3-8B GQA",
        "value": round(ms_step, 4),
        "unit": "ms/layer",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": (f"synthetic: AR(1) keys rho=0.9 sigma=0.44 + RoPE base 5e5, Gaussian Q/V, "
                 f"seed {args.seed}; Euclidean tau={tau:.4f} calibrated to r={ratio:g} "
                 f"(realised {r_real:.3f}) in the {arith} selection arithmetic, chunk 512, W={W}"),
        "config": {"workload": (f"config{args.config}: delta prefill attention, one layer, "
                                f"B={B} Hq={Hq} Hkv={Hkv} D={D} N={N} {args.dtype} causal r={ratio:g}"),
                   "seq_len": N, "global_batch": B, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(hyb_tflops, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(hyb_tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": traffic_bytes(args, N, r_real, ratio),
                     "kernel": "attn_w64_kernel<hybrid> (da_hybrid_prefill)",
                     "algorithmic_flops": fl["algorithmic"],
                     "executed_tile_flops": fl["executed_tiles"]},
    }
    rec.update({k2: v2 for k2, v2 in res.items()
                if k2 not in ("seq_len", "hybrid_algorithmic_flops", "hybrid_executed_tile_flops")})
    res["record"] = rec
    res["cpu_inputs"] = (q.cpu(), k.cpu(), v.cpu(), tau)
    return res


def run_only(args):
    """``--only``: one part of the config-1/2 layer for K launches (rocprofv3 captures)."""
    import torch
    from deltaattention_amd import ops, synth
    N = args.seq or (32768 if args.config == 1 else 131072)
    W = args.window
    q, k, v = layer_inputs(args, N)
    tau, r_real = synth.calibrate_threshold(k, args.ratio, arith=args.select_arith)
    keep, _ = ops.select(k, tau, 512, arith=args.select_arith)
    packed = ops.pack(keep, k, v)
    out = torch.empty_like(q)
    fns = {
        "delta": lambda: ops.delta_prefill(q, k, v, tau, 512, window=W, arith=args.select_arith),
        "hybrid": lambda: ops.hybrid_prefill(q, k, v, packed.k_packed, packed.v_packed,
                                             packed.timestamps, packed.counts, window=W,
                                             num_packed_dev=packed.num_packed, out=out),
        "dense": lambda: ops.dense_prefill(q, k, v, causal=True, out=out),
        "compress": lambda: ops.pack(ops.select(k, tau, 512, arith=args.select_arith)[0], k, v, out=packed),
    }
    if args.only == "copy":
        src = torch.randint(0, 1000, (1 << 29,), dtype=torch.int16, device=q.device)  # 1 GiB
        dst = torch.empty_like(src)
        fns["copy"] = lambda: dst.copy_(src)
    if args.only == "convert":
        src = torch.randn(1 << 28, dtype=torch.float32, device=q.device)  # 1 GiB read
        dst = torch.empty(1 << 28, dtype=torch.bfloat16, device=q.device)  # 512 MiB written
        fns["convert"] = lambda: dst.copy_(src)
    fn = fns[args.only]
    for _ in range(args.warmup):
        fn()
    ms = time_loop(fn, args.steps)
    print(f"only={args.only} N={N} r={r_real:.3f} steps={args.steps} ms/launch={ms:.4f}", flush=True)


if __name__ == "__main__":
    main()
