"""Benchmark of the grafted-SwiGLU layer path on one MI355X.

Workload (one step): the Llama-3-8B-shape grafted MLP layer with bf16
weights/activations and fp32 accumulation -- hidden 4096, base intermediate
14336, one appended graft slice of 1024 neurons, 8 x 2048 = 16384 tokens --
    RMSNorm fwd (eps 1e-5) -> grafted MLP fwd -> graft-only MLP bwd (dX and
    per-slice dW) from an f32 upstream gradient -> RMSNorm bwd -> AdamW on
    the graft params (lr 1e-4, betas 0.9/0.999, wd 0.01, global clip 1.0).
Inputs are synthetic (weights ~N(0,0.02), x ~N(0,1), gamma ~1+N(0,0.02),
dy ~N(0,1) in f32 as the reference's backward receives it), drawn on the GPU
and resident in HBM before timing.

Also measured: shadow_bake materialising 32 layers of baked [15360,4096] /
[4096,15360] matrices (GB/s against HBM), the HBM-bound kernels, attention,
the decoder layer, one shadow-eval batch (LM head and eval statistics at
16384 x 128256), and the reference's graft math in PyTorch on a bounded
token sample on the host cores (cpu_baseline).

Prints ONE JSON line. Usage: python bench.py [--steps K] [--warmup W]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "graft MLP fwd+bwd tokens/sec @Llama-3-8B shape; % bf16 MFMA peak; bake GB/s"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (published)
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E (published)

M, D, I, S = 16384, 4096, 14336, 1024
N = I + S
EPS = 1e-5
LR, B1, B2, AEPS, WD = 1e-4, 0.9, 0.999, 1e-8, 0.01
CLIP = 1.0  # the reference's per-step global gradient clip (src/config.hpp:85)

# algorithmic work per launch (FLOP) of each GEMM kernel of one step
GEMM_FLOP = {
    "gate_up": 2 * M * D * 2 * N,   # gate + up over N = I + S neurons
    "down": 2 * M * N * D,          # K-concat of base and graft columns
    "dinter": 2 * M * D * N,        # dInter with the SiLU*up derivative epilogue
    "dx": 2 * M * 2 * N * D,        # concat-K over [dgate | dup]
    "wgrad": 3 * 2 * S * D * M,     # dW gate/up/down of the slice (one launch)
}
STEP_FLOP = sum(GEMM_FLOP.values())
# algorithmic HBM bytes per launch of the bandwidth-bound kernels
HBM_BYTES = {
    "rmsnorm_fwd": 2 * M * D * 2 + D * 2 + M * 4,          # x in, y out (bf16), gamma, mean-square out
    "rmsnorm_bwd": M * D * (4 + 2 + 4) + D * 2 + M * 4,    # dy f32, x bf16 in, dx f32 out, gamma, mean-square
    # the slice's three projections in one launch: w, g, m, v in; w, m, v
    # out; the four bf16 mirrors out
    "adamw_pack": 3 * S * D * (4 * 4 + 3 * 4 + 4 * 2),
    # the clip's sum of squares over the three projections' gradients
    "clip_sumsq": 3 * S * D * 4,
    # the backward's operand layout pass: x (bf16) and the f32 upstream
    # gradient in; the gradient rounded to bf16 (row-major) and x and the
    # gradient transposed into the MFMA fragment layout out
    "shuffle_tr": M * D * (2 + 4) + 3 * M * D * 2,
    # the three graft slices of dgate, dup and inter transposed for the
    # weight-gradient GEMMs (read and written once)
    "transpose16": 3 * M * S * 2 * 2,
}
ROPE_B, ROPE_T, ROPE_HQ, ROPE_HK, ROPE_HD, ROPE_THETA = 2, 4096, 32, 8, 128, 500000.0
# masked cross-entropy bench: 4 x 4096 tokens, Llama-3 vocabulary
CE_B, CE_T, CE_V = 4, 4096, 128256


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--no-bake", action="store_true", help="skip the shadow_bake measurement")
    ap.add_argument("--no-layer", action="store_true", help="skip the decoder-layer measurement")
    ap.add_argument("--layer-only", action="store_true",
                    help="only the attention kernel and decoder-layer measurements (for profiling them alone)")
    ap.add_argument("--no-eval", action="store_true", help="skip the shadow-eval (LM head + eval statistics) line")
    ap.add_argument("--eval-only", action="store_true",
                    help="only the shadow-eval measurement (for profiling it alone)")
    ap.add_argument("--cpu-tokens", type=int, default=4096)
    ap.add_argument("--vendor", action="store_true",
                    help="only the step's GEMM shapes on torch's bf16 GEMMs (hipBLASLt) beside this library's "
                         "kernels in the same run, outside the timed step")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (scale for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from glt_amd import _ffi as F, synth

    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    lib = F.load()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    bf = torch.bfloat16
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None

    def fill(t, seed, tid, mean, std):
        F.call("glt_fill_normal", p(t), F.DTYPE_BF16 if t.dtype == bf else F.DTYPE_F32, t.numel(), seed, tid,
               mean, std, sp)
        return t

    log("[bench] drawing inputs")
    x_raw = fill(torch.empty((M, D), dtype=bf, device=dev), synth.SEED_X, synth.TID_X, 0.0, 1.0)
    gamma = fill(torch.empty(D, dtype=bf, device=dev), synth.SEED_GAMMA, synth.TID_GAMMA, 1.0, 0.02)
    dy = fill(torch.empty((M, D), dtype=torch.float32, device=dev), synth.SEED_DY, synth.TID_DY, 0.0, 1.0)
    wg = fill(torch.empty((I, D), dtype=bf, device=dev), synth.SEED_BASE, synth.TID_GATE, 0.0, 0.02)
    wu = fill(torch.empty((I, D), dtype=bf, device=dev), synth.SEED_BASE, synth.TID_UP, 0.0, 0.02)
    wd = fill(torch.empty((D, I), dtype=bf, device=dev), synth.SEED_BASE, synth.TID_DOWN, 0.0, 0.02)
    masters = fill(torch.empty(3 * S * D, dtype=torch.float32, device=dev), 1, 1, 0.0, 0.02)
    packed = torch.empty(lib.glt_graft_packed_size(S, D), dtype=torch.uint8, device=dev)

    sl = (F.GraftSlice * 1)()
    sl[0] = F.GraftSlice(I, S, 0, D, masters.data_ptr(), masters.data_ptr() + 4 * S * D,
                         masters.data_ptr() + 8 * S * D, packed.data_ptr())
    desc = F.MlpDesc(M, D, I, N, F.DTYPE_BF16, F.MLP_EXPLICIT | F.MLP_DY_F32, 1, sl, None)
    prepared = torch.empty(lib.glt_base_prepared_size(ctypes.byref(desc)), dtype=torch.uint8, device=dev)
    F.call("glt_base_prepare", ctypes.byref(desc), p(wg), p(wu), p(wd), p(prepared), sp)
    F.call("glt_graft_pack", sl, p(packed), sp)
    base = F.BaseWeights(wg.data_ptr(), wu.data_ptr(), wd.data_ptr(), prepared.data_ptr())

    x = torch.empty((M, D), dtype=bf, device=dev)
    var = torch.empty(M, dtype=torch.float32, device=dev)
    y = torch.empty((M, D), dtype=bf, device=dev)
    g = torch.empty((M, N), dtype=bf, device=dev)
    u = torch.empty((M, N), dtype=bf, device=dev)
    inter = torch.empty((M, N), dtype=bf, device=dev)
    dx = torch.empty((M, D), dtype=torch.float32, device=dev)
    dx_raw = torch.empty((M, D), dtype=torch.float32, device=dev)
    grads = torch.zeros(3 * S * D, dtype=torch.float32, device=dev)
    adam_m = torch.zeros(3 * S * D, dtype=torch.float32, device=dev)
    adam_v = torch.zeros(3 * S * D, dtype=torch.float32, device=dev)
    gg = (F.GraftGrads * 1)()
    gg[0] = F.GraftGrads(grads.data_ptr(), grads.data_ptr() + 4 * S * D, grads.data_ptr() + 8 * S * D)
    ws_bytes = lib.glt_mlp_bwd_workspace_size(ctypes.byref(desc))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    gptr = F.ptr_array([grads.data_ptr()])
    mptr, vptr = F.ptr_array([adam_m.data_ptr()]), F.ptr_array([adam_v.data_ptr()])
    pkptr = F.ptr_array([packed.data_ptr()])
    clip_ws_bytes = lib.glt_adamw_workspace_size(0)
    clip_ws = torch.empty(clip_ws_bytes, dtype=torch.uint8, device=dev)

    def step(i):
        F.call("glt_rmsnorm_fwd", p(x_raw), p(gamma), p(x), p(var), M, D, EPS, sp)
        F.call("glt_mlp_fwd", ctypes.byref(desc), ctypes.byref(base), p(x), p(y), p(g), p(u), p(inter), sp)
        # graft-only backward and the RMSNorm's backward (the latter on the
        # CUs the weight-gradient GEMM leaves idle)
        F.call("glt_mlp_rmsnorm_bwd", ctypes.byref(desc), ctypes.byref(base), p(x), p(dy), p(g), p(u), p(inter),
               p(dx), gg, p(ws), ws_bytes, p(x_raw), p(gamma), p(var), EPS, p(dx_raw), sp)
        F.call("glt_adamw_graft_step", sl, 1, gptr, mptr, vptr, pkptr, 7, i, LR, B1, B2, AEPS, WD, CLIP, p(clip_ws),
               clip_ws_bytes, sp)

    if args.eval_only:
        print(json.dumps({"shadow_eval": bench_shadow_eval(torch, F, sp, p)}), flush=True)
        return
    if args.layer_only:
        out = {"attention": bench_attention(torch, F, sp, p),
               "decoder_layer": bench_layer(torch, F, lib, dev, sp, p, fill, base, sl)}
        print(json.dumps(out), flush=True)
        return

    log("[bench] warmup")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    if args.vendor:
        print(json.dumps({"vendor_gemm": bench_vendor(torch, F, step, args, x, dy, wg, wu, wd, masters, inter)}),
              flush=True)
        return

    # timed region: K steps between events on the launch stream
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    log(f"[bench] {ms_step:.3f} ms/step")

    # per-kernel durations: the same steps again with launch timing on
    F.call("glt_profile_enable", 1)
    for i in range(args.steps):
        step(args.warmup + args.steps + i)
    torch.cuda.synchronize()
    prof = F.profile_collect()
    F.call("glt_profile_enable", 0)
    kernels = {k: {"avg_ms": tot / cnt, "launches_per_step": cnt / args.steps} for k, (tot, cnt) in prof.items()}
    for k, v in kernels.items():
        v["ms_per_step"] = v["avg_ms"] * v["launches_per_step"]
        if k in GEMM_FLOP:  # per-step FLOP over per-step time of that kernel
            v["tflops"] = GEMM_FLOP[k] / (v["ms_per_step"] * 1e-3) / 1e12
            v["mfma_frac"] = v["tflops"] / PEAK_BF16_TFLOPS
    gemm_ms = sum(kernels[k]["ms_per_step"] for k in GEMM_FLOP if k in kernels)

    # One GPU's share of an 8-way token-parallel step: the same step on the
    # first M / 8 tokens of the same buffers (rows are contiguous), with the
    # same graft weights and optimizer state. The multi-GPU step would add
    # the all-reduce of the graft gradients, which is not run here.
    m_share = M // 8
    desc_share = F.MlpDesc(m_share, D, I, N, F.DTYPE_BF16, F.MLP_EXPLICIT | F.MLP_DY_F32, 1, sl, None)
    assert lib.glt_mlp_bwd_workspace_size(ctypes.byref(desc_share)) <= ws_bytes

    def step_share(i):
        F.call("glt_rmsnorm_fwd", p(x_raw), p(gamma), p(x), p(var), m_share, D, EPS, sp)
        F.call("glt_mlp_fwd", ctypes.byref(desc_share), ctypes.byref(base), p(x), p(y), p(g), p(u), p(inter), sp)
        F.call("glt_mlp_rmsnorm_bwd", ctypes.byref(desc_share), ctypes.byref(base), p(x), p(dy), p(g), p(u),
               p(inter), p(dx), gg, p(ws), ws_bytes, p(x_raw), p(gamma), p(var), EPS, p(dx_raw), sp)
        F.call("glt_adamw_graft_step", sl, 1, gptr, mptr, vptr, pkptr, 7, i, LR, B1, B2, AEPS, WD, CLIP, p(clip_ws),
               clip_ws_bytes, sp)

    for i in range(args.warmup):
        step_share(i)
    torch.cuda.synchronize()
    ev0.record(stream)
    for i in range(args.steps):
        step_share(args.warmup + i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_share = ev0.elapsed_time(ev1) / args.steps
    share = {"tokens": m_share, "ms_per_step": round(ms_share, 4),
             "tokens_per_s": round(m_share / (ms_share * 1e-3), 1),
             "mfma_frac": round(STEP_FLOP / 8 / (ms_share * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
             "note": "one GPU's share of an 8-way token-parallel step of the same workload; the gradient "
                     "all-reduce of the multi-GPU step is not run"}
    log(f"[bench] 1/8 share ({m_share} tokens): {ms_share:.3f} ms/step")
    dom = max((k for k in kernels if k in GEMM_FLOP), key=lambda k: kernels[k]["ms_per_step"])
    dom_flop = GEMM_FLOP[dom] / kernels[dom]["launches_per_step"]  # per launch
    achieved = dom_flop / (kernels[dom]["avg_ms"] * 1e-3) / 1e12
    # HBM bytes per launch are not measured in this run: hardware counters
    # need a rocprofv3 --pmc run of their own. The figure is that run's
    # (profiles/traffic_<kernel>.json, FETCH_SIZE and WRITE_SIZE passes
    # scaled by a copy of known size; commands in
    # profiles/mlp_step_llama3_8b_traffic.md), labelled as such.
    traffic, traffic_source = None, None
    tf = os.path.join(ROOT, "profiles", f"traffic_{dom}.json")
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("hbm_bytes_per_launch")
        traffic_source = (f"profiles/traffic_{dom}.json: separate rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs "
                          f"of this bench (commands in profiles/mlp_step_llama3_8b_traffic.md), not this run")
    roofline = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "traffic_source": traffic_source, "flop_per_launch": dom_flop}

    # HBM-bound kernels against the HBM roofline. RMSNorm, the clip, the
    # layout passes and the AdamW update: their launches in the step above
    # (so in the step's own cache state), each timed by HIP events bound to
    # its dispatch (hipExtLaunchKernelGGL: the kernel's execution time, as a
    # kernel trace reports it). RoPE at the decoder-layer shape (2 x 4096
    # tokens, 32 q / 8 kv heads of 128, theta 5e5): one launch at a time,
    # after a read of a 1 GiB buffer that leaves none of its inputs in the
    # caches (the 256 MB last-level cache would otherwise hold the whole
    # input across repeated launches).
    # The step's RMSNorm backward runs beside the weight-gradient GEMM on
    # the CUs that launch leaves idle (label rmsnorm_bwd_beside), so its
    # duration there says nothing about bandwidth: glt_rmsnorm_bwd is timed
    # on its own over the step's buffers.
    F.call("glt_profile_enable", 1)
    for _ in range(args.steps):
        F.call("glt_rmsnorm_bwd", p(dx), p(x_raw), p(gamma), p(var), p(dx_raw), M, D, EPS, sp)
    torch.cuda.synchronize()
    tot, cnt = F.profile_collect().get("rmsnorm_bwd", (0.0, 1))
    F.call("glt_profile_enable", 0)
    rms_bwd_alone = tot / cnt
    hbm = {}
    for k, nbytes in HBM_BYTES.items():
        if k == "rmsnorm_bwd":
            t = rms_bwd_alone
            hbm[k] = {"bytes": nbytes, "ms": round(t, 5), "GB_per_s": round(nbytes / (t * 1e-3) / 1e9, 1),
                      "frac_hbm": round(nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                      "timing": "kernel duration, launched alone on the step's buffers (in the step it runs "
                                "beside the weight-gradient GEMM)"}
            continue
        if k in kernels:
            t = kernels[k]["avg_ms"]
            hbm[k] = {"bytes": nbytes, "ms": round(t, 5), "GB_per_s": round(nbytes / (t * 1e-3) / 1e9, 1),
                      "frac_hbm": round(nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                      "timing": "kernel duration in the step (events bound to the dispatch)"}
    flush_buf = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    flush_buf.fill_(1.0)
    flush_out = torch.empty((), dtype=torch.float32, device=dev)

    def cold_ms(fn, label, reps=20):
        # each launch after a 1 GiB read; its duration from the launch timing
        # (events bound to the kernel dispatch)
        fn()
        torch.cuda.synchronize()
        F.call("glt_profile_enable", 1)
        for _ in range(reps):
            torch.sum(flush_buf, 0, out=flush_out)
            fn()
        torch.cuda.synchronize()
        tot, cnt = F.profile_collect().get(label, (0.0, 1))
        F.call("glt_profile_enable", 0)
        return tot / cnt

    hbm["rope"] = bench_rope(torch, F, sp, p, cold_ms)
    hbm["masked_ce"] = bench_masked_ce(torch, F, sp, p)
    hbm["torch_copy"] = bench_copy(torch)
    del flush_buf, flush_out
    attention = bench_attention(torch, F, sp, p)
    shadow_eval = None if args.no_eval else bench_shadow_eval(torch, F, sp, p)
    layer = None
    if not args.no_layer:
        layer = bench_layer(torch, F, lib, dev, sp, p, fill, base, sl)

    # shadow_bake: 32 layers materialised (config 4)
    bake = None
    if not args.no_bake:
        bake = bench_bake(torch, F, lib, dev, sp, p)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, args.cpu_tokens, wg, wu, wd, masters, x_raw, gamma, dy)

    out = {
        "metric": METRIC,
        "value": round(M / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "Llama-3-8B-shape grafted SwiGLU MLP layer: RMSNorm + graft-only fwd+bwd (f32 upstream gradient) + clipped AdamW",
                   "tokens": M, "hidden": D, "base_intermediate": I, "graft_slice": S, "parallelism": "none (1 GPU)"},
        "step_mfma_frac": round(STEP_FLOP / (ms_step * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "gemm_mfma_frac": round(STEP_FLOP / (gemm_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        # the fwd+bwd GEMM path alone (sum of the step's GEMM launches), beside
        # the full step of "value"
        "gemm_path": {"ms": round(gemm_ms, 4), "tokens_per_s": round(M / (gemm_ms * 1e-3), 1)},
        "dp8_share": share,
        "roofline": roofline,
        "hbm_kernels": hbm,
        "cpu_baseline": cpu,
        "bake": bake,
        "attention": attention,
        "shadow_eval": shadow_eval,
        "decoder_layer": layer,
        "kernels": {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in sorted(kernels.items())},
    }
    print(json.dumps(out), flush=True)


def bench_vendor(torch, F, step, args, x, dy, wg, wu, wd, masters, inter, reps=10):
    """The step's GEMM shapes on torch's bf16 GEMMs (hipBLASLt on this image)
    next to this library's kernels from the same run (launch timing of the
    step's own launches). Operands: the step's inputs where they exist (x,
    the weights with the graft rows appended, the saved inter, dy rounded to
    bf16); the dX GEMM's [dgate | dup] operand is drawn ~N(0, 0.01). Each
    entry states what each side writes: the library's gate/up and dInter
    GEMMs carry their epilogues (SiLU*up with three outputs; the SiLU*up
    derivative reading two saved arrays and writing two), torch's write one
    plain output."""
    F.call("glt_profile_enable", 1)
    for i in range(args.steps):
        step(1000 + i)
    torch.cuda.synchronize()
    prof = F.profile_collect()
    F.call("glt_profile_enable", 0)
    ours = {k: tot / cnt for k, (tot, cnt) in prof.items()}
    bf = torch.bfloat16
    gd = masters[:S * D].view(S, D).to(bf)
    ud = masters[S * D:2 * S * D].view(S, D).to(bf)
    dd = masters[2 * S * D:].view(S, D).to(bf)
    w_gu = torch.cat([wg, gd, wu, ud], 0)                  # [2N, D]
    w_down = torch.cat([wd, dd.t()], 1).contiguous()       # [D, N]
    w_down_t = w_down.t().contiguous()                     # [N, D]
    w_dx = torch.cat([wg, gd, wu, ud], 0)                  # [2N, D]: dX = [dg | du] . w_dx
    dyb = dy.to(bf)
    dgdu = torch.empty((M, 2 * N), dtype=bf, device=x.device).normal_(0.0, 0.01)
    try:
        torch.mm(dyb[:64], w_down[:, :64], out_dtype=torch.float32)
        dx_f32 = True
    except Exception:   # no mixed-output mm in this torch build
        dx_f32 = False
    cases = {
        "gate_up": (lambda: torch.nn.functional.linear(x, w_gu), "[M, 2N] bf16 = %d B" % (M * 2 * N * 2),
                    "inter, gate_pre, up_pre [M, N] bf16 = %d B (SiLU*up epilogue)" % (3 * M * N * 2)),
        "down": (lambda: torch.nn.functional.linear(inter, w_down), "[M, D] bf16 = %d B" % (M * D * 2),
                 "[M, D] bf16 = %d B" % (M * D * 2)),
        "dinter": (lambda: torch.nn.functional.linear(dyb, w_down_t), "[M, N] bf16 = %d B" % (M * N * 2),
                   "dgate, dup [M, N] bf16 = %d B, reading gate_pre, up_pre = %d B (SiLU*up derivative)"
                   % (2 * M * N * 2, 2 * M * N * 2)),
        "dx": ((lambda: torch.mm(dgdu, w_dx, out_dtype=torch.float32)) if dx_f32 else (lambda: torch.mm(dgdu, w_dx)),
               "[M, D] %s = %d B" % (("f32", M * D * 4) if dx_f32 else ("bf16", M * D * 2)),
               "[M, D] f32 = %d B" % (M * D * 4)),
    }
    out = {}
    stream = torch.cuda.current_stream()
    for k, (fn, tb, ob) in cases.items():
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / reps
        o = ours.get(k)
        out[k] = {"flop": GEMM_FLOP[k], "torch_ms": round(t, 4), "torch_tflops": round(GEMM_FLOP[k] / t / 1e9, 1),
                  "torch_writes": tb, "ours_ms": round(o, 4) if o else None,
                  "ours_tflops": round(GEMM_FLOP[k] / o / 1e9, 1) if o else None, "ours_writes": ob}
        log(f"[bench] {k}: torch {t:.3f} ms, ours {o:.3f} ms")
    out["note"] = ("torch times are back-to-back launches between events on the stream; ours are the step's "
                   "launches timed by events bound to each dispatch")
    return out


def bench_rope(torch, F, sp, p, cold_ms):
    """RoPE in place on q [2,4096,32*128] and k [2,4096,8*128] bf16 (the
    decoder-layer shape); algorithmic bytes: q and k read and written."""
    bf = torch.bfloat16
    q = torch.empty((ROPE_B, ROPE_T, ROPE_HQ * ROPE_HD), dtype=bf, device="cuda")
    k = torch.empty((ROPE_B, ROPE_T, ROPE_HK * ROPE_HD), dtype=bf, device="cuda")
    for i, t in enumerate((q, k)):
        F.call("glt_fill_normal", p(t), F.DTYPE_BF16, t.numel(), 400, i, 0.0, 1.0, sp)

    def run():
        F.call("glt_rope_fwd", p(q), ROPE_HQ, p(k), ROPE_HK, ROPE_B, ROPE_T, ROPE_HD, ROPE_THETA, 0, sp)

    t = cold_ms(run, "rope")
    nbytes = 2 * 2 * ROPE_B * ROPE_T * (ROPE_HQ + ROPE_HK) * ROPE_HD
    return {"bytes": nbytes, "ms": round(t, 5), "GB_per_s": round(nbytes / (t * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "timing": "kernel duration (events bound to the dispatch), each launch after a 1 GiB read"}


def bench_shadow_eval(torch, F, sp, p, reps=3):
    """The shadow-eval batch at 4 x 4096 tokens of the Llama-3 vocabulary:
    the LM head (logits = x . lm_head^T, 16384 x 4096 x 128256, bf16, MFMA in
    row blocks of under 2 GiB of logits) and then the eval statistics on those
    logits (CE sum and count, logit sum and sum of squares, and the
    reference's FNV-1a hash chained over every logit byte). The statistics
    pass reads the logits once (HBM-bound); the exact hash's three passes
    (low-nibble maps, high-nibble maps, affine) are bound by their integer
    arithmetic, so the line reports their time, not an HBM fraction."""
    B, T, V = CE_B, CE_T, CE_V
    M, Dm = B * T, D
    lib = F.load()
    x = torch.empty((M, Dm), dtype=torch.bfloat16, device="cuda")
    head = torch.empty((V, Dm), dtype=torch.bfloat16, device="cuda")
    F.call("glt_fill_normal", p(x), F.DTYPE_BF16, x.numel(), 502, 0, 0.0, 1.0, sp)
    F.call("glt_fill_normal", p(head), F.DTYPE_BF16, head.numel(), 503, 0, 0.0, 0.05, sp)
    prepared = torch.empty(lib.glt_lm_head_prepared_size(V, Dm), dtype=torch.uint8, device="cuda")
    F.call("glt_lm_head_prepare", p(head), V, Dm, p(prepared), sp)
    logits = torch.empty((B, T, V), dtype=torch.bfloat16, device="cuda")
    ids = torch.randint(0, V, (B, T), dtype=torch.int32, device="cuda")
    nbytes_ws = lib.glt_eval_stats_workspace_size(B, T)
    ws = torch.empty(nbytes_ws, dtype=torch.uint8, device="cuda")
    res = F.EvalResult()

    def run():
        F.call("glt_lm_head_fwd", p(x), M, Dm, p(head), p(prepared), V, p(logits), sp)
        F.call("glt_eval_stats", p(logits), V, p(ids), B, T, V, F.EVAL_HASH_REFERENCE, F.FNV_BASIS, ctypes.byref(res),
               p(ws), nbytes_ws, sp)

    run()
    torch.cuda.synchronize()
    F.call("glt_profile_enable", 1)
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    prof = F.profile_collect()
    F.call("glt_profile_enable", 0)
    ms = lambda pred: sum(tot for k, (tot, cnt) in prof.items() if pred(k)) / reps
    t_head = ms(lambda k: k == "lm_head")
    t_stats = ms(lambda k: k == "eval_rows")
    t_hash = ms(lambda k: k.startswith("eval_hash"))
    flop = 2.0 * M * Dm * V
    nbytes = 2 * M * V
    del logits, prepared, head, x
    return {"rows": M, "vocab": V, "hidden": Dm,
            "lm_head": {"flop": flop, "ms": round(t_head, 4), "tflops": round(flop / (t_head * 1e-3) / 1e12, 1),
                        "mfma_frac": round(flop / (t_head * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)},
            "stats_pass": {"bytes": nbytes, "ms": round(t_stats, 4),
                           "GB_per_s": round(nbytes / (t_stats * 1e-3) / 1e9, 1),
                           "frac_hbm": round(nbytes / (t_stats * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)},
            "exact_hash_ms": round(t_hash, 4),
            "eval_stats_ms": round(t_stats + t_hash, 4),
            "hash_bound": "integer arithmetic (16 runs of the low-byte chain per logit in two passes, one 64-bit run)"}


def bench_masked_ce(torch, F, sp, p, reps=5):
    """Masked cross-entropy + grad_logits over 4 x 4096 tokens of the
    Llama-3 vocabulary (128256), bf16 logits, every 3rd token excluded;
    algorithmic bytes: logits read once, gradient written once."""
    B, T, V = CE_B, CE_T, CE_V
    bf = torch.bfloat16
    logits = torch.empty((B, T, V), dtype=bf, device="cuda")
    grad = torch.empty_like(logits)
    F.call("glt_fill_normal", p(logits), F.DTYPE_BF16, logits.numel(), 500, 0, 0.0, 3.0, sp)
    ids = torch.randint(0, V, (B, T), dtype=torch.int32, device="cuda")
    ood = torch.zeros((B, T), dtype=torch.int32, device="cuda")
    ood[:, 1::3] = 1
    stats = torch.empty(4, dtype=torch.float32, device="cuda")
    nbytes_ws = F.load().glt_masked_ce_workspace_size(B, T)
    ws = torch.empty(nbytes_ws, dtype=torch.uint8, device="cuda")

    def run():
        F.call("glt_masked_ce", p(logits), V, p(ids), p(ood), B, T, V, 1.0, p(grad), V, None, p(stats), p(ws),
               nbytes_ws, sp)

    run()
    torch.cuda.synchronize()
    F.call("glt_profile_enable", 1)
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    tot, cnt = F.profile_collect().get("masked_ce", (0.0, 1))
    F.call("glt_profile_enable", 0)
    t = tot / cnt
    nbytes = 2 * 2 * B * T * V
    del logits, grad
    return {"bytes": nbytes, "ms": round(t, 4), "GB_per_s": round(nbytes / (t * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4), "tokens": B * T, "vocab": V}


def bench_attention(torch, F, sp, p, reps=10):
    """Causal GQA attention forward at the decoder-layer shape (q [2,4096,32,128],
    k/v [2,4096,8,128] bf16); algorithmic work 4*B*Hq*T^2*hd/2 (two causal
    products). The time is the call's: the V transpose into the workspace
    and the attention kernel."""
    bf = torch.bfloat16
    q = torch.empty((ROPE_B, ROPE_T, ROPE_HQ, ROPE_HD), dtype=bf, device="cuda")
    k = torch.empty((ROPE_B, ROPE_T, ROPE_HK, ROPE_HD), dtype=bf, device="cuda")
    v = torch.empty_like(k)
    o = torch.empty_like(q)
    for i, t in enumerate((q, k, v)):
        F.call("glt_fill_normal", p(t), F.DTYPE_BF16, t.numel(), 500, i, 0.0, 1.0, sp)
    nb = F.load().glt_attention_workspace_size(ROPE_B, ROPE_T, ROPE_HK, ROPE_HD)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")

    def run():
        F.call("glt_attention_fwd", p(q), p(k), p(v), p(o), ROPE_B, ROPE_T, ROPE_HQ, ROPE_HK, ROPE_HD,
               ROPE_HD ** -0.5, 1, p(ws), nb, sp)

    run()
    torch.cuda.synchronize()
    F.call("glt_profile_enable", 1)
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    prof = F.profile_collect()
    F.call("glt_profile_enable", 0)
    tot, cnt = prof.get("attention", (0.0, 1))
    vt, vcnt = prof.get("attn_vt", (0.0, 1))
    t = tot / cnt + vt / vcnt
    flop = 4 * ROPE_B * ROPE_HQ * ROPE_T * ROPE_T * ROPE_HD // 2
    return {"flop": flop, "ms": round(t, 5), "kernel_ms": round(tot / cnt, 5), "v_transpose_ms": round(vt / vcnt, 5),
            "tflops": round(flop / (t * 1e-3) / 1e12, 1),
            "mfma_frac": round(flop / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}


def bench_layer(torch, F, lib, dev, sp, p, fill, base, sl, reps=5):
    """Decoder layer with the grafted MLP at 2 x 4096 tokens (hidden 4096, 32
    query / 8 kv heads of 128, base intermediate 14336, one appended 1024
    slice): glt_layer_fwd, then the graft-only backward of the MLP with
    recompute (glt_mlp_bwd); base weights random, the MLP's shared with the
    MLP step. The backward recomputes the gate/up pre-activations (the
    reference's recompute_ffn) and computes the input gradient dX of the
    MLP as well as the graft gradients. Work: the step's GEMM formulas at
    8192 tokens plus the recompute (one more gate/up GEMM), attention
    projections 2*M*D*(2*q width + 2*kv width), SDPA 4*B*Hq*T^2*hd/2."""
    bf = torch.bfloat16
    B, T = ROPE_B, ROPE_T
    Mt, nq, nk = B * T, ROPE_HQ * ROPE_HD, ROPE_HK * ROPE_HD
    wq = fill(torch.empty((nq, D), dtype=bf, device=dev), 600, 1, 0.0, 0.02)
    wk = fill(torch.empty((nk, D), dtype=bf, device=dev), 600, 2, 0.0, 0.02)
    wv = fill(torch.empty((nk, D), dtype=bf, device=dev), 600, 3, 0.0, 0.02)
    wo = fill(torch.empty((D, nq), dtype=bf, device=dev), 600, 4, 0.0, 0.02)
    ln_in = fill(torch.empty(D, dtype=bf, device=dev), 600, 5, 1.0, 0.02)
    ln_post = fill(torch.empty(D, dtype=bf, device=dev), 600, 6, 1.0, 0.02)
    x = fill(torch.empty((Mt, D), dtype=bf, device=dev), 600, 7, 0.0, 1.0)
    dy = fill(torch.empty((Mt, D), dtype=torch.float32, device=dev), 600, 8, 0.0, 1.0)
    md = F.MlpDesc(Mt, D, I, N, F.DTYPE_BF16, F.MLP_EXPLICIT, 1, sl, None)
    ld = F.LayerDesc(B, T, ROPE_HQ, ROPE_HK, ROPE_HD, ROPE_THETA, EPS, md)
    lw = F.LayerWeights(p(wq), p(wk), p(wv), p(wo), p(ln_in), p(ln_post), None, base)
    prep = torch.empty(lib.glt_attn_prepared_size(ctypes.byref(ld)), dtype=torch.uint8, device=dev)
    lw.prepared = prep.data_ptr()
    F.call("glt_attn_prepare", ctypes.byref(ld), ctypes.byref(lw), p(prep), sp)
    fws = torch.empty(lib.glt_layer_fwd_workspace_size(ctypes.byref(ld)), dtype=torch.uint8, device=dev)
    x_ffn = torch.empty_like(x)
    var = torch.empty(Mt, dtype=torch.float32, device=dev)
    bd = F.MlpDesc(Mt, D, I, N, F.DTYPE_BF16, F.MLP_EXPLICIT | F.MLP_RECOMPUTE | F.MLP_DY_F32, 1, sl, None)
    bws = torch.empty(lib.glt_mlp_bwd_workspace_size(ctypes.byref(bd)), dtype=torch.uint8, device=dev)
    grads = torch.zeros(3 * S * D, dtype=torch.float32, device=dev)
    dx = torch.empty((Mt, D), dtype=torch.float32, device=dev)
    gg = (F.GraftGrads * 1)()
    gg[0] = F.GraftGrads(grads.data_ptr(), grads.data_ptr() + 4 * S * D, grads.data_ptr() + 8 * S * D)

    def fwd():
        F.call("glt_layer_fwd", ctypes.byref(ld), ctypes.byref(lw), p(x), p(x_ffn), p(var), None, None, None,
               p(fws), fws.numel(), sp)

    def bwd():
        F.call("glt_mlp_bwd", ctypes.byref(bd), ctypes.byref(base), p(x_ffn), p(dy), None, None, None, p(dx), gg,
               p(bws), bws.numel(), sp)

    fwd()
    bwd()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record()
    for _ in range(reps):
        fwd()
    ev[1].record()
    for _ in range(reps):
        bwd()
    ev[2].record()
    torch.cuda.synchronize()
    t_f, t_b = ev[0].elapsed_time(ev[1]) / reps, ev[1].elapsed_time(ev[2]) / reps
    mlp_flop = (STEP_FLOP + GEMM_FLOP["gate_up"]) * Mt // M
    attn_flop = 2 * Mt * D * (2 * nq + 2 * nk) + 4 * B * ROPE_HQ * T * T * ROPE_HD // 2
    ms = t_f + t_b
    return {"workload": "decoder layer (2 x 4096 tokens, 32/8 heads, grafted MLP) fwd + the MLP's graft-only bwd "
                        "(recompute, dX and the graft gradients)",
            "tokens": Mt, "ms_fwd": round(t_f, 4), "ms_bwd": round(t_b, 4), "ms_step": round(ms, 4),
            "tokens_per_s": round(Mt / (ms * 1e-3), 1), "algorithmic_flop": mlp_flop + attn_flop,
            "mfma_frac": round((mlp_flop + attn_flop) / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}


def bench_copy(torch, nbytes=1 << 30, reps=10):
    """Device-to-device copy of 1 GiB with torch's copy kernel (bytes = read
    + write), reported beside the HBM-bound kernels as a familiar yardstick;
    it is not the hardware ceiling (a one-16-byte-chunk-per-thread
    nontemporal copy streams faster)."""
    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / reps
    del src, dst
    return {"bytes": 2 * nbytes, "ms": round(t, 5), "GB_per_s": round(2 * nbytes / (t * 1e-3) / 1e9, 1),
            "frac_hbm": round(2 * nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}


def calibrate_copy(torch, nbytes=1 << 30, reps=3):
    """A plain device-to-device copy of nbytes, reps times: the reference
    kernel whose FETCH_SIZE / WRITE_SIZE (known to be nbytes each) scales
    the counter readings of the path's kernels."""
    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes": nbytes, "reps": reps}), flush=True)


def bench_bake(torch, F, lib, dev, sp, p, L=32, reps=5):
    """Config 4: base gate/up [14336,4096] and down [4096,14336] bf16 plus a
    1024-neuron bf16 graft per layer, materialised into [15360,4096] /
    [4096,15360] for 32 layers. Algorithmic bytes: read base + read graft +
    write baked."""
    bf = torch.bfloat16
    log("[bench] bake: allocating 32 layers")
    bases = [[torch.empty(sh, dtype=bf, device=dev) for sh in ((I, D), (I, D), (D, I))] for _ in range(L)]
    outs = [[torch.empty(sh, dtype=bf, device=dev) for sh in ((N, D), (N, D), (D, N))] for _ in range(L)]
    grafts = [torch.empty(3 * S * D, dtype=bf, device=dev) for _ in range(L)]
    for l in range(L):
        for q, t in enumerate(bases[l]):
            F.call("glt_fill_normal", p(t), F.DTYPE_BF16, t.numel(), 0, 1000 + 3 * l + q, 0.0, 0.02, sp)
        F.call("glt_fill_normal", p(grafts[l]), F.DTYPE_BF16, grafts[l].numel(), 1, 2000 + l, 0.0, 0.02, sp)
    pl = (ctypes.c_int32 * 4)(I, S, 0, D)
    gp = F.ptr_array([t.data_ptr() for t in grafts])
    desc = F.BakeDesc(F.BAKE_MATERIALIZE, L, 0, L - 1, 7, D, I, N, F.DTYPE_BF16, 1, pl, gp)
    arrs = [F.ptr_array([bases[l][q].data_ptr() for l in range(L)]) for q in range(3)]
    oarrs = [F.ptr_array([outs[l][q].data_ptr() for l in range(L)]) for q in range(3)]

    def run():
        st = F.ModelState(0)
        F.call("glt_shadow_bake", ctypes.byref(desc), ctypes.byref(st), arrs[0], arrs[1], arrs[2], oarrs[0],
               oarrs[1], oarrs[2], sp)

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    F.call("glt_profile_enable", 1)
    run()
    torch.cuda.synchronize()
    prof = F.profile_collect()
    F.call("glt_profile_enable", 0)
    nbytes = L * 3 * 2 * (I * D + S * D + N * D)
    kern_ms = prof.get("bake", (ms, 1))[0]
    del bases, outs, grafts
    torch.cuda.empty_cache()
    return {"layers": L, "bytes": nbytes, "ms": round(ms, 4), "GB_per_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "kernel_ms": round(kern_ms, 4), "launches": prof.get("bake", (0, 0))[1]}


def _torch_cpu_step(torch, x_raw, gamma, Wg, Wu, Wd, masters, dy, adam):
    """One step of the grafted layer in PyTorch on the CPU: the reference's
    explicit-injection graft math with ATen ops, in the config's dtype where
    the reference is bf16 and in f32 where it is f32:
    RMSNorm (grafting.hip:116-146); base gate/up F.linear in bf16 (at::linear,
    src/layer_forward_impl.inc:72, :122); the slice's f32 expand output of
    bf16 operands injected into the bf16 pre-activations (appended slice:
    onto zero base rows, src/kernels_elementwise_impl.inc:314-326); SiLU*up;
    base down in bf16 plus the f32 contract term; the graft-only backward with
    the f32 base GEMMs against f32 weight copies and bf16 graft GEMMs
    (src/layer_backward_impl.inc:45-361); RMSNorm backward
    (src/kernels_rmsnorm_kernels.inc:70-126); AdamW on the f32 masters
    (src/kernels_optimizer_impl.inc:27-51). Masters are updated in place."""
    F_ = torch.nn.functional
    bf = torch.bfloat16
    Dg, Du, Dd = masters
    x = x_raw.float()
    var = x.pow(2).mean(-1, keepdim=True)
    r = torch.rsqrt(var + EPS)
    w = gamma.float()
    xn = (x * r * w).to(bf)
    xf = xn.float()
    dgb, dub, ddb = (t.to(bf).float() for t in (Dg, Du, Dd))
    g = torch.cat([F_.linear(xn, Wg), (xf @ dgb.t()).to(bf)], 1).float()
    u = torch.cat([F_.linear(xn, Wu), (xf @ dub.t()).to(bf)], 1).float()
    inter = (F_.silu(g) * u).to(bf)
    _y = (F_.linear(inter[:, :I], Wd).float() + inter[:, I:].float() @ ddb).to(bf)
    # graft-only backward
    dyf = dy.float()
    dyb = dy.to(bf).float()
    gi = torch.cat([dyf @ Wd.float(), dyb @ ddb.t()], 1)
    grad_d = inter[:, I:].float().t() @ dyb
    sg = torch.sigmoid(g)
    dg = gi * u * sg * (1 + g * (1 - sg))
    du = gi * g * sg
    dgs, dus = dg[:, I:].to(bf).float(), du[:, I:].to(bf).float()
    grad_g, grad_u = dgs.t() @ xf, dus.t() @ xf
    dxn = dg[:, :I] @ Wg.float() + du[:, :I] @ Wu.float() + dgs @ dgb + dus @ dub
    mean = (dxn * x * w).mean(-1, keepdim=True)
    dx_raw = dxn * r * w - x * mean * r.pow(3)
    for p_, grad_, (m_, v_) in zip((Dg, Du, Dd), (grad_g, grad_u, grad_d), adam):
        m_.mul_(B1).add_(grad_, alpha=1 - B1)
        v_.mul_(B2).addcmul_(grad_, grad_, value=1 - B2)
        p_.sub_(LR * (m_ / (1 - B1)) / ((v_ / (1 - B2)).sqrt() + AEPS) + LR * WD * p_)
    return dx_raw


def cpu_baseline(torch, T, wg, wu, wd, masters, x_raw, gamma, dy):
    """The grafted layer step in PyTorch on the host cores (bf16, the
    config's dtype), on the first T tokens of the same synthetic inputs:
    RMSNorm, grafted MLP forward, graft-only backward, RMSNorm backward,
    AdamW. One warmup step, then the median of three."""
    import platform
    import subprocess
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    log(f"[bench] cpu baseline: PyTorch CPU on {T} tokens, {torch.get_num_threads()} threads")
    c = lambda t: t.detach().cpu()
    Wg, Wu, Wd, gm = c(wg), c(wu), c(wd), c(gamma)
    ms = c(masters).reshape(3, S, D).clone()
    xr, dyy = c(x_raw[:T]), c(dy[:T])
    adam = [(torch.zeros(S, D), torch.zeros(S, D)) for _ in range(3)]
    times = []
    for rep in range(4):
        t0 = time.perf_counter()
        _torch_cpu_step(torch, xr, gm, Wg, Wu, Wd, [ms[0], ms[1], ms[2]], dyy, adam)
        if rep:
            times.append(time.perf_counter() - t0)
    dt = sorted(times)[1]
    cpu_model = platform.processor()
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                cpu_model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return {"value": round(T / dt, 2), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{T} of the {M} tokens of one step (RMSNorm, grafted MLP fwd, graft-only bwd, RMSNorm bwd, "
                      f"AdamW), median of 3 steps {dt:.2f} s; PyTorch {torch.__version__} CPU in bf16, "
                      f"{torch.get_num_threads()} threads (os.cpu_count() = {threads}) on {cpu_model}"}


if __name__ == "__main__":
    main()
