#!/usr/bin/env python3
"""Decode benchmark: greedy tok/s at bs=1 on the Qwen3.5-2B-shaped hybrid decoder (Q8F weights,
seeded random init), plus the Q8F matvec bandwidth against the 8 TB/s HBM roofline.

Workload: 24 layers (18 Gated DeltaNet + 6 gated GQA), hidden 2048, FFN 6144, vocab 248320,
tied embeddings, random-init weights N(0, 0.02) quantised to Q8F, seed 0; a 512-token uniform
random prompt is fed through the decode step, then W untimed and K timed greedy decode steps.  A
"step" is one token through the whole model (embedding -> 24 layers -> final norm -> lm_head ->
argmax) with weights and caches resident in HBM, run by the persistent step kernel (--chunk steps
per launch; each step's argmax feeds the next step on the device).

Prints one JSON line.  Only one GPU is used; --gpus N > 1 exits with a message.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen-3.5_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PUBLISHED_TOKS = 43.0  # README.md:11-13,22 of the reference (RTX 4060 Ti, wgpu, real weights)


def q8_bytes(N, K, M):
    """Algorithmic HBM bytes of one Q8F matvec: int8 W + f32 scales + f32 x + f32 y."""
    return K * N + 4 * K * N // 64 + 4 * M * K + 4 * M * N


def step_bytes(d, ctx):
    """Algorithmic bytes of one decode step at context ctx (weights + states + KV)."""
    H, F, V = d.hidden, d.ffn, d.vocab
    nh, vd = d.lin_heads, d.lin_heads * d.lin_dv
    conv_dim = 2 * nh * d.lin_dk + vd
    ah, kvh, hd = d.attn_heads, d.kv_heads, d.head_dim
    n_full = sum(1 for l in range(d.n_layers) if (l + 1) % d.full_interval == 0)
    n_lin = d.n_layers - n_full
    mv = 0
    mv += n_lin * (q8_bytes(conv_dim + vd, H, 1) + q8_bytes(H, vd, 1) + 2 * H * nh * 4)
    mv += n_full * (q8_bytes(ah * hd * 2 + 2 * kvh * hd, H, 1) + q8_bytes(H, ah * hd, 1))
    mv += d.n_layers * (q8_bytes(2 * F, H, 1) + q8_bytes(H, F, 1))
    mv += q8_bytes(V, H, 1)
    state = n_lin * (2 * nh * d.lin_dk * d.lin_dv * 4 + 2 * conv_dim * 3 * 4 + conv_dim * 4 * 4)
    kv = n_full * (2 * kvh * ctx * hd * 4)
    return mv + state + kv


def time_lm_head(torch, q35, m, d, reps):
    """Average duration of the lm_head Q8F matvec (kernels.rs q8_lm_head) with HIP events on the
    stream it is launched on, using the model's tied embedding table."""
    lib = q35.lib()
    eq, _ = m.tensor_ptr("embed_tokens.q")
    es, _ = m.tensor_ptr("embed_tokens.scale")
    hv = torch.randn(d.hidden, device="cuda")
    h = hv.data_ptr()
    W = q35._lib.Q8F(eq, es, d.vocab, d.hidden, q35.Q35_NK)
    logits = torch.empty(d.vocab, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    for _ in range(3):
        q35._lib.check(lib.q35_q8_lm_head(h, 1, W, logits.data_ptr(), s.cuda_stream))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        q35._lib.check(lib.q35_q8_lm_head(h, 1, W, logits.data_ptr(), s.cuda_stream))
    e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps  # us


def matvec_sweep(torch, q35, m, d, reps=4):
    """Per-shape KN matvec rate over the model's own weights, rotating through all layers so the
    working set (> 256 MB) exceeds the MALL; events around back-to-back launches (so the figure
    includes the ~1.6 us launch gap of each kernel)."""
    lib = q35.lib()
    shapes = {
        "mlp.gate_proj [6144x2048]": ("mlp.gate_proj", d.ffn, d.hidden, range(d.n_layers)),
        "mlp.down_proj [2048x6144]": ("mlp.down_proj", d.hidden, d.ffn, range(d.n_layers)),
        "linear_attn.in_proj_qkv [6144x2048]": ("linear_attn.in_proj_qkv", 6144, d.hidden,
                                                 [l for l in range(d.n_layers) if (l + 1) % 4]),
        "linear_attn.out_proj [2048x2048]": ("linear_attn.out_proj", d.hidden, 2048,
                                              [l for l in range(d.n_layers) if (l + 1) % 4]),
        "self_attn.q_proj [4096x2048]": ("self_attn.q_proj", 4096, d.hidden,
                                         [l for l in range(d.n_layers) if (l + 1) % 4 == 0]),
        "self_attn.k_proj [512x2048]": ("self_attn.k_proj", 512, d.hidden,
                                        [l for l in range(d.n_layers) if (l + 1) % 4 == 0]),
    }
    x = torch.randn(max(d.hidden, d.ffn), device="cuda")
    y = torch.empty(max(d.ffn, 8192), device="cuda")
    ws = q35.workspace(1 << 24, key="bench_gemv")
    s = torch.cuda.current_stream()
    out = {}
    for label, (name, N, K, layers) in shapes.items():
        descs = []
        for l in layers:
            q, _ = m.tensor_ptr(f"layers.{l}.{name}.q")
            sc, _ = m.tensor_ptr(f"layers.{l}.{name}.scale")
            descs.append(q35._lib.Q8F(q, sc, K, N, q35.Q35_KN_TILED))
        for W in descs:
            q35._lib.check(lib.q35_q8_gemv(x.data_ptr(), 1, W, y.data_ptr(), ws.data_ptr(), ws.numel(), s.cuda_stream))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            for W in descs:
                q35._lib.check(lib.q35_q8_gemv(x.data_ptr(), 1, W, y.data_ptr(), ws.data_ptr(), ws.numel(),
                                               s.cuda_stream))
        e1.record(s)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(descs))
        gbs = q8_bytes(N, K, 1) / us / 1e3
        out[label] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                      "working_set_MB": round(len(descs) * q8_bytes(N, K, 1) / 1e6, 1)}
    return out


def copy_calibration():
    """Three device-to-device copies of exactly 1 GiB: what FETCH_SIZE / WRITE_SIZE report for a
    known byte count, the scale factor for the step kernel's counters."""
    import torch
    torch.cuda.set_device(0)
    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print("copied 3 x 1 GiB", flush=True)


# HBM traffic of one step_kernel<2> launch of 64 steps in this workload: FETCH_SIZE + WRITE_SIZE
# per dispatch from two rocprofv3 --pmc passes over `bench.py --no-cpu --no-sweep`, scaled by the
# counters' reading for a 1 GiB copy (`bench.py --copy-calibration`): x2.0 and x1.0.  Measured for
# the kernel at the commit that recorded it; profiles/step_kernel_decode_2b_traffic.md has the
# commands and the per-dispatch values.
STEP_TRAFFIC_PER_LAUNCH = 139.72e9


def cpu_baseline(q35, d, prompt, budget_s=20.0):
    """Oracle (CPU restatement) decode tok/s on the host cores, bounded sample."""
    import oracle as O
    t0 = time.time()
    ref = O.Model(O.cfg_from_dims(d), lambda name, n: q35.synth_model_tensor(d, 0, name, n), 64)
    build_s = time.time() - t0
    tok = int(prompt[0])
    for t in prompt[:2]:
        tok, _, _ = ref.step(int(t))
    t1 = time.time()
    tok, _, _ = ref.step(tok)
    one = time.time() - t1
    n = max(2, min(32, int(budget_s / max(one, 1e-3))))
    t1 = time.time()
    for _ in range(n):
        tok, _, _ = ref.step(tok)
    el = time.time() - t1
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(n / el, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} greedy decode steps of the full 2B-shaped model after a 3-token prefill, "
                      f"oracle/oracle.c (OpenMP, x86-64-v3), weights built in {build_s:.0f}s (not timed)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-sweep", action="store_true", help="skip the per-shape matvec sweep")
    ap.add_argument("--chunk", type=int, default=64, help="decode steps per persistent-kernel launch")
    ap.add_argument("--readback", action="store_true",
                    help="also time one launch per token with a host readback each step (main.rs loop)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run three 1 GiB device copies (reference point for FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the decode path is single-GPU; multi-GPU is "
              "design-only), so --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import q35

    torch.cuda.set_device(0)
    d = q35.dims_2b()
    chunk = args.chunk
    n_pre = -(-args.prompt // chunk) * chunk
    n_warm = -(-args.warmup // chunk) * chunk
    n_timed = -(-args.steps // chunk) * chunk
    tmax = n_pre + n_warm + n_timed + 8
    t0 = time.time()
    m = q35.TextForCausalLM(d, seed=args.seed, tmax=tmax)
    create_s = time.time() - t0
    grid = m.persistent_grid()
    prompt = np.random.default_rng(args.seed).integers(0, d.vocab, n_pre).astype(np.int32)
    st = torch.cuda.Stream()  # a stream of its own (the null stream's handle would mean "model stream")
    torch.cuda.set_stream(st)
    sh = st.cuda_stream

    # The prompt goes through the decode step; every persistent launch below is `chunk` steps, so
    # the kernel's average launch duration in a profile of this command is the timed one.
    t0 = time.time()
    m.generate(prompt[:chunk], 0, mode="persistent", stream=sh)
    for c0 in range(chunk, n_pre, chunk):
        m.generate(prompt[c0:c0 + chunk], 0, mode="persistent", stream=sh)
    m.check(stream=sh)
    prefill_s = time.time() - t0
    for _ in range(n_warm // chunk):
        m.decode(chunk, mode="persistent", stream=sh)
    m.check(stream=sh)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_timed // chunk)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in ev:
        e0.record(st)
        m.decode(chunk, mode="persistent", stream=sh)
        e1.record(st)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    m.check(stream=sh)
    launch_ms = [e0.elapsed_time(e1) for e0, e1 in ev]
    kern_s = sum(launch_ms) * 1e-3
    toks = n_timed / el
    ms = el * 1e3 / n_timed
    ctx0 = n_pre + n_warm
    bytes_timed = sum(step_bytes(d, ctx0 + i + 1) for i in range(n_timed))
    bytes_per_launch = bytes_timed / len(ev)
    avg_launch_us = kern_s * 1e6 / len(ev)
    achieved = bytes_per_launch / (avg_launch_us * 1e-6) / 1e9
    hist = m.tensor("hist", np.int32)[:ctx0 + n_timed]

    toks_readback = None
    if args.readback:  # main.rs semantics: one launch per token, token read back and synced each step
        m.reset()
        m.generate(prompt[:chunk], 0, mode="persistent", stream=sh)
        _, dec_s = m.generate(prompt[chunk:chunk + 1], 64, mode="persistent", readback_each=True, stream=sh)
        toks_readback = 64 / dec_s

    lm_us = time_lm_head(torch, q35, m, d, reps=50)
    lm_bytes = q8_bytes(d.vocab, d.hidden, 1)
    lm_gbs = lm_bytes / lm_us / 1e3
    sweep = None if args.no_sweep else matvec_sweep(torch, q35, m, d)
    m.close()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(q35, d, prompt)

    line = {
        "metric": "decode tok/s bs=1 Qwen3.5-2B-shape Q8F; matvec HBM GB/s vs 8 TB/s peak",
        "value": round(toks, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(toks / PUBLISHED_TOKS, 2),
        "dtype": "f32",
        "data": "synthetic (random-init weights N(0,0.02) quantised to Q8F, seed 0; uniform random prompt)",
        "config": {"workload": "greedy decode bs=1, Qwen3.5-2B-shaped hybrid decoder (18 Gated DeltaNet + 6 gated "
                               "GQA layers, hidden 2048, FFN 6144, vocab 248320, tied Q8F embeddings)",
                   "batch": 1, "prompt_len": n_pre, "ctx_range": [ctx0, ctx0 + n_timed],
                   "weights": "int8 Q8F per-64 f32 scales",
                   "launch": f"persistent step kernel, {chunk} steps per launch, grid {grid}x512"},
        "roofline": {"kernel": f"step_kernel<2>: persistent decode step, {chunk} tokens per launch",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": STEP_TRAFFIC_PER_LAUNCH if chunk == 64 else None,
                     "bytes_per_launch": int(bytes_per_launch), "avg_launch_us": round(avg_launch_us, 1)},
        "lm_head_kernel": {"kernel": "nk_kernel<1,2>: standalone Q8F lm_head 248320x2048 (kernels.rs q8_lm_head)",
                           "achieved_GBs": round(lm_gbs, 1), "frac": round(lm_gbs / HBM_PEAK_GBS, 4),
                           "avg_launch_us": round(lm_us, 2)},
        "greedy_ids_checksum": int(np.sum(hist.astype(np.int64) * (np.arange(hist.size) % 9973 + 1)) % 1000000007),
        "tok_s_with_readback": None if toks_readback is None else round(toks_readback, 2),
        "prefill_tok_s_via_decode_step": round(args.prompt / prefill_s, 1),
        "model_build_s": round(create_s, 1),
        "matvec_kn_sweep": sweep,
        "cpu_baseline": cpu,
        "vs_baseline_note": "published ~43 tok/s is the reference's custom-kernel decode on an RTX 4060 Ti",
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
