"""Benchmark of the MI355X backend on the GWP-0.5-shaped MoT hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads (synthetic, seeded, random-init weights; inputs resident in HBM
before the timed region):
  chunk  (default) one GWP-0.5-shaped MoT action chunk: prompt projection,
         prefix pass over 1 state + 3x1024 visual tokens with 512 prompt
         tokens, 10 flow-matching denoise steps of the 48-token action
         expert; 30 layers, d=3072, 24x128 heads, FFN 14336, both experts.
  ffn    one dense FFN block at 2048 tokens: LayerNorm+adaLN modulation ->
         W_up [14336x3072] + bias + GELU-tanh -> W_down [3072x14336] + bias +
         gated residual (bf16 hidden state, fp32 accumulation).
  gemm   one MUL_MAT: W bf16 [3072x3072], X f32 [256x3072] -> Y f32.
  decode the action-expert decode against a cached prefix (--batch B chunks):
         the 10-step unrolled denoise graph of B independent chunks, each 48
         action queries over its own resident bf16 KV (1 state + 3072 visual
         self-attention keys and 512 prompt keys per layer, 30 layers, 24x128),
         the projections on 48*B rows.

Prints one JSON line (rank 0) with roofline and cpu_baseline objects.  The
dominant kernel's duration is measured with HIP events on the backend's
stream; rocprofv3 summaries of the same command are kept under profiles/.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
for sub in ("wam.cpp_amd", "oracle"):
    sys.path.insert(0, str(REPO / sub))

import wamx  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def cpu_info():
    cores = os.cpu_count() or 1
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return cores, model


def _normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0, bf16: bool = False) -> np.ndarray:
    """Seeded synthetic data (f32, or bf16 bit patterns when bf16=True)."""
    v = np.random.default_rng(seed).standard_normal(n, dtype=np.float32) * np.float32(std) + np.float32(mean)
    return wamx.f32_to_bf16(v) if bf16 else v


# HBM bytes per launch of the roofline kernels, from the rocprofv3 FETCH_SIZE /
# WRITE_SIZE passes of `bench.py --probe-traffic`, each scaled by the factor
# the same counter gives for a streaming kernel of known size.  The summary in
# profiles/ holds one "traffic_bytes <key> <bytes>" line per kernel.
TRAFFIC_FILE = REPO / "profiles" / "traffic_roofline_kernels.md"


def measured_traffic(key: str):
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            f = line.strip().strip("`").split()
            if len(f) == 3 and f[0] == "traffic_bytes" and f[1] == key:
                return float(f[2])
    except OSError:
        pass
    return None


def time_op(be, fn, reps: int) -> float:
    """Average ms of fn() over reps launches, HIP events on the backend stream."""
    t = wamx.Timer(be)
    fn()
    be.sync()
    t.start()
    for _ in range(reps):
        fn()
    return t.stop_ms() / reps


# ---------------------------------------------------------------------------
def workload_gemm(be, args):
    M, K, N = 3072, 3072, 256
    w = _normal(M * K, 0x5EED0000 + 1, 0.0, 0.02, bf16=True)
    x = _normal(N * K, 0x5EED0000 + 2)
    dw, dx, dy = be.array(w), be.array(x), be.empty(N * M * 4)

    def step():
        wamx.check(be.lib.wamx_op_mul_mat(be.ptr, dw.ptr, K, dx.ptr, wamx.TYPE_F32, K, dy.ptr, wamx.TYPE_F32, M,
                                          M, N, K), "mul_mat")

    flops = 2.0 * M * N * K
    bytes_ = M * K * 2 + N * K * 4 + N * M * 4
    for _ in range(args.warmup):
        step()
    be.sync()
    t = wamx.Timer(be)
    t.start()
    for _ in range(args.steps):
        step()
    ms = t.stop_ms() / args.steps
    roof = {"bound": "hbm", "achieved": bytes_ / (ms * 1e-3) / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": bytes_ / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, "traffic": None,
            "kernel": "gemm_tile<128,128> (f32 activations)", "tflops": flops / (ms * 1e-3) / 1e12}
    # CPU baseline: the oracle's MUL_MAT on the full problem.
    import oracle
    t0 = time.perf_counter()
    oracle.mul_mat(w.reshape(M, K), x.reshape(N, K))
    cpu_ms = (time.perf_counter() - t0) * 1e3
    cores, model = cpu_info()
    cpu = {"value": cpu_ms, "unit": "ms per MUL_MAT", "cores": oracle.num_threads(), "kind": "port",
           "sample": f"full 3072x3072x256 MUL_MAT on {model} ({cores} logical CPUs)"}
    return {"metric": "ms per MUL_MAT (3072x3072 bf16 weight, 256 f32 tokens)", "unit": "ms", "value": ms,
            "ms_per_step": ms, "higher_is_better": False, "dtype": "bf16",
            "config": {"workload": "single MUL_MAT W[3072x3072] bf16 x X[256x3072] f32", "tokens": N},
            "roofline": roof, "cpu_baseline": cpu}


def workload_ffn(be, args):
    T, D, F = 2048, 3072, 14336
    seed = 0x5EED0000 + 2
    x = _normal(T * D, seed + 1, 0.0, 1.0, bf16=True)
    shift = _normal(D, seed + 2, 0.0, 0.1)
    scale = _normal(D, seed + 3, 0.0, 0.1)
    gate = _normal(D, seed + 4, 0.0, 0.1)
    w_up = _normal(F * D, seed + 5, 0.0, 0.02, bf16=True)
    b_up = _normal(F, seed + 6, 0.0, 0.02, bf16=True)
    w_dn = _normal(D * F, seed + 7, 0.0, 0.02, bf16=True)
    b_dn = _normal(D, seed + 8, 0.0, 0.02, bf16=True)
    dx, dsh, dsc, dg = be.array(x), be.array(shift), be.array(scale), be.array(gate)
    dwu, dbu, dwd, dbd = be.array(w_up), be.array(b_up), be.array(w_dn), be.array(b_dn)
    dn, dh, dout = be.empty(T * D * 2), be.empty(T * F * 2), be.empty(T * D * 2)
    lib = be.lib

    def norm():
        wamx.check(lib.wamx_op_norm_modulation_bf16(be.ptr, dx.ptr, D, dsc.ptr, dsh.ptr, 0, dn.ptr, T, D, 1e-6))

    def up():
        wamx.check(lib.wamx_op_linear(be.ptr, dwu.ptr, dn.ptr, wamx.TYPE_BF16, dbu.ptr, wamx.EPI_BIAS_GELU, None,
                                      None, dh.ptr, F, T, D))

    def down():
        wamx.check(lib.wamx_op_linear(be.ptr, dwd.ptr, dh.ptr, wamx.TYPE_BF16, dbd.ptr, wamx.EPI_BIAS_GATED, dx.ptr,
                                      dg.ptr, dout.ptr, D, T, F))

    def step():
        norm()
        up()
        down()

    for _ in range(args.warmup):
        step()
    be.sync()
    t = wamx.Timer(be)
    t.start()
    for _ in range(args.steps):
        step()
    ms = t.stop_ms() / args.steps
    gemm_flops = 2.0 * T * D * F
    up_ms = time_op(be, up, 10)
    down_ms = time_op(be, down, 10)
    norm_ms = time_op(be, norm, 20)
    dom_ms, dom = (up_ms, "gemm_dma_pipe (FFN up + bias + GELU)") if up_ms >= down_ms else \
        (down_ms, "gemm_dma_pipe (FFN down + bias + gated residual)")
    roof = {"bound": "mfma", "achieved": gemm_flops / (dom_ms * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": gemm_flops / (dom_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, "traffic": None,
            "kernel": dom, "kernel_ms": dom_ms,
            "kernels_ms": {"norm_mod_bf16": norm_ms, "ffn_up": up_ms, "ffn_down": down_ms},
            "norm_gbs": (2 * T * D * 2) / (norm_ms * 1e-3) / 1e9}
    # CPU baseline: the oracle's FFN block on 256 of the 2048 tokens, scaled x8.
    import oracle
    ts = 256
    xs = x.reshape(T, D)[:ts]
    t0 = time.perf_counter()
    n = oracle.norm_mod_bf16(xs, scale, shift, 1e-6)
    h = oracle.linear(w_up.reshape(F, D), n, b_up, oracle.EPI_BIAS_GELU)
    oracle.linear(w_dn.reshape(D, F), h, b_dn, oracle.EPI_BIAS_GATED, xs, gate)
    cpu_ms = (time.perf_counter() - t0) * 1e3 * (T / ts)
    cores, model = cpu_info()
    cpu = {"value": cpu_ms, "unit": "ms per FFN block", "cores": oracle.num_threads(), "kind": "port",
           "sample": f"{ts} of {T} tokens, scaled x{T // ts}, on {model} ({cores} logical CPUs)"}
    return {"metric": "ms per dense FFN block (2048 tokens, 3072->14336->3072, bf16)", "unit": "ms", "value": ms,
            "ms_per_step": ms, "higher_is_better": False, "dtype": "bf16",
            "config": {"workload": "dense FFN block: LN+adaLN, W_up[14336x3072]+GELU, W_down[3072x14336]+gated "
                                   "residual, 2048 tokens", "tokens": T, "gemm_tflops": gemm_flops * 2 / (ms * 1e-3) / 1e12},
            "roofline": roof, "cpu_baseline": cpu}


def _gwp_inputs(cfg, seed):
    A, T = cfg["action_dim"], cfg["action_chunk"]
    return (_normal(A, seed + 1), _normal(cfg["z_dim"] * 4 * cfg["grid_h"] * cfg["grid_w"], seed + 2),
            _normal(cfg["n_lang"] * cfg["t5_hidden"], seed + 3), _normal(T * A, seed + 4))


def _read_weights(be, m, keep):
    out = {}
    lib = be.lib
    for i in range(lib.wamx_gwp_n_weights(m)):
        name = lib.wamx_gwp_weight_name(m, i).decode()
        if not keep(name):
            continue
        t = lib.wamx_gwp_weight(m, name.encode())
        n = lib.wamx_nelements(t)
        a = np.empty(n, np.uint16)
        wamx.check(lib.wamx_backend_tensor_get(t, a.ctypes.data, 0, n * 2), name)
        out[name] = a
    return out


def workload_chunk(be, args):
    """Full synthetic GWP-0.5-shaped action chunk: prompt projection, prefix
    pass over 1 state + 3x1024 visual tokens with 512 prompt tokens, then 10
    flow-matching denoise steps of the 48-token action expert, 30 layers at
    width 3072 (24x128 heads, FFN 14336) in both experts."""
    import ctypes as C
    lib = be.lib
    c = lib.wamx_gwp_default_config()
    cfg = {k: getattr(c, k) for k, _ in wamx.GwpConfig._fields_}
    m = lib.wamx_gwp_create(be.ptr, C.byref(c))
    if not m:
        raise RuntimeError(wamx.last_error())
    wamx.check(lib.wamx_gwp_init_synthetic(m, 0x5EED0003, 0.02), "init_synthetic")
    state, latent, prompt, noise = _gwp_inputs(cfg, 0x5EED0003)
    wamx.check(lib.wamx_gwp_set_inputs(m, state.ctypes.data, latent.ctypes.data, prompt.ctypes.data,
                                       noise.ctypes.data), "set_inputs")
    tm = wamx.GwpTiming()
    for _ in range(max(1, args.warmup)):
        wamx.check(lib.wamx_gwp_predict(m, None), "predict")
    be.sync()
    phases = np.zeros(3)
    action = np.empty(noise.size, np.float32)
    # One request at a time, as the reference's predict serves them: submit
    # the three graphs, then read the action chunk back (which waits for it).
    t = wamx.Timer(be)
    t.start()
    for _ in range(args.steps):
        wamx.check(lib.wamx_gwp_predict(m, None), "predict")
        wamx.check(lib.wamx_gwp_get_action(m, action.ctypes.data), "get_action")
    ms = t.stop_ms() / args.steps
    # Back-to-back chunks with no read-back between them, for comparison.
    t.start()
    for _ in range(args.steps):
        wamx.check(lib.wamx_gwp_predict(m, None), "predict")
    ms_pipelined = t.stop_ms() / args.steps
    # Whole requests including the host inputs' upload (state, latent, prompt,
    # noise: 10.75 MB of f32 through wamx_gwp_set_inputs), as the reference's
    # predict uploads them per request (cache.cpp:428-439, mot.cpp:565-588).
    # Host-to-device copies are not part of `value` (inputs resident in HBM).
    t0 = time.perf_counter()
    for _ in range(args.steps):
        wamx.check(lib.wamx_gwp_set_inputs(m, state.ctypes.data, latent.ctypes.data, prompt.ctypes.data,
                                           noise.ctypes.data), "set_inputs")
        wamx.check(lib.wamx_gwp_predict(m, None), "predict")
        wamx.check(lib.wamx_gwp_get_action(m, action.ctypes.data), "get_action")
    ms_with_upload = (time.perf_counter() - t0) * 1e3 / args.steps
    upload_bytes = 4 * (state.size + latent.size + prompt.size + noise.size)
    # The same requests with the projected-prompt cache on, as the reference's
    # wam-bench --mode steady runs them (apps/wam-bench.cpp:83): after the
    # first request the prompt upload and the prompt graphs are skipped
    # (cache.cpp:53-67).  Reported beside `value`, which projects every
    # request's prompt (--mode raw).
    wamx.check(lib.wamx_gwp_set_prompt_cache(m, 4), "set_prompt_cache")
    wamx.check(lib.wamx_gwp_set_inputs(m, state.ctypes.data, latent.ctypes.data, prompt.ctypes.data,
                                       noise.ctypes.data), "set_inputs")
    wamx.check(lib.wamx_gwp_predict(m, None), "predict")
    wamx.check(lib.wamx_gwp_get_action(m, action.ctypes.data), "get_action")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        wamx.check(lib.wamx_gwp_set_inputs(m, state.ctypes.data, latent.ctypes.data, prompt.ctypes.data,
                                           noise.ctypes.data), "set_inputs")
        wamx.check(lib.wamx_gwp_predict(m, None), "predict")
        wamx.check(lib.wamx_gwp_get_action(m, action.ctypes.data), "get_action")
    ms_steady = (time.perf_counter() - t0) * 1e3 / args.steps
    hits, misses = C.c_uint64(), C.c_uint64()
    wamx.check(lib.wamx_gwp_prompt_cache_stats(m, C.byref(hits), C.byref(misses)), "prompt_cache_stats")
    if hits.value != args.steps:
        raise RuntimeError(f"projected-prompt cache: {hits.value} hits in {args.steps} repeated requests")
    wamx.check(lib.wamx_gwp_set_prompt_cache(m, 0), "set_prompt_cache")
    for _ in range(3):
        wamx.check(lib.wamx_gwp_predict(m, C.byref(tm)), "predict")
        phases += np.array([tm.prompt_ms, tm.prefix_ms, tm.denoise_ms]) / 3
    wamx.check(lib.wamx_gwp_get_action(m, action.ctypes.data), "get_action")
    if not np.all(np.isfinite(action)):
        raise RuntimeError("non-finite action chunk")
    params = int(lib.wamx_gwp_param_count(m))
    nodes = [int(lib.wamx_gwp_graph_nodes(m, i)) for i in range(3)]

    # Dominant kernel: the visual FFN-up GEMM of the prefix pass (3072 tokens x
    # W[14336 x 3072], bias + GELU epilogue), timed standalone on the stream.
    T, D, F = cfg["grid_h"] * cfg["grid_w"], cfg["hidden"], cfg["ffn_dim"]
    w_up = lib.wamx_gwp_weight(m, b"gwp.blocks.0.visual_expert.ffn.net.0.proj.weight")
    b_up = lib.wamx_gwp_weight(m, b"gwp.blocks.0.visual_expert.ffn.net.0.proj.bias")
    dx = be.array(_normal(T * D, 5, 0.0, 1.0, bf16=True))
    dy = be.empty(T * F * 2)

    def up():
        wamx.check(lib.wamx_op_linear(be.ptr, w_up.contents.data, dx.ptr, wamx.TYPE_BF16, b_up.contents.data,
                                      wamx.EPI_BIAS_GELU, None, None, dy.ptr, F, T, D), "linear")
    # Timed as it runs in the chunk: one launch right after a request
    # (wamx_gwp_predict) on the backend stream, HIP events around it, so the
    # GPU is in the clock and power state the chunk leaves it in; 10 such
    # launches averaged.  Back to back, the MFMAs stay busy for milliseconds
    # and the power-limited clock sinks launch by launch (236 -> 304 us over
    # 20 launches); that sustained figure is reported beside it.
    up_ms_sustained = time_op(be, up, 20)
    t_up, post = wamx.Timer(be), []
    for _ in range(10):
        wamx.check(lib.wamx_gwp_predict(m, None), "predict")
        t_up.start()
        up()
        post.append(t_up.stop_ms())
    up_ms = float(np.mean(post))
    flops = 2.0 * T * D * F
    # The 48-token FFN-up of the action expert (HBM-bound weight streaming),
    # cycling through the 30 layers' weights as the denoise pass does, so the
    # 88 MB weight is not resident in the 256 MB last-level cache.
    Ta, Da, Fa = cfg["action_chunk"], cfg["action_hidden"], cfg["action_ffn_dim"]
    aups = [(lib.wamx_gwp_weight(m, f"gwp.blocks.{l}.action_expert.ffn.net.0.proj.weight".encode()),
             lib.wamx_gwp_weight(m, f"gwp.blocks.{l}.action_expert.ffn.net.0.proj.bias".encode()))
            for l in range(cfg["n_layers"])]
    dxa = be.array(_normal(Ta * Da, 6, 0.0, 1.0, bf16=True))
    dya = be.empty(Ta * Fa * 2)
    nxt = [0]

    def aup():
        w_aup, b_aup = aups[nxt[0] % len(aups)]
        nxt[0] += 1
        wamx.check(lib.wamx_op_linear_tiled(be.ptr, w_aup.contents.data, dxa.ptr, wamx.TYPE_BF16,
                                            b_aup.contents.data, wamx.EPI_BIAS_GELU, None, None, dya.ptr, Fa, Ta, Da),
                   "linear_tiled")
    aup_ms = time_op(be, aup, 60)
    aup_bytes = Fa * Da * 2 + Ta * Da * 2 + Ta * Fa * 2 + Fa * 2
    roof = {"bound": "mfma", "achieved": flops / (up_ms * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": flops / (up_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, "traffic": measured_traffic("gemm_dma_ffn_up"),
            "kernel": "gemm_dma_pipe<256,224, MFMA 16x16x32>: prefix visual FFN-up 3072 tok x [14336 x 3072] + bias + GELU",
            "kernel_ms": up_ms, "timing": "one launch after each of 10 requests (the chunk's clock state)",
            "kernel_ms_sustained": up_ms_sustained,
            "frac_sustained": flops / (up_ms_sustained * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, "flops_per_launch": flops,
            "algorithmic_bytes": T * D * 2 + F * D * 2 + F * 2 + T * F * 2,
            "skinny": {"kernel": "gemm_skinny_wk: denoise FFN-up 48 tok x [14336 x 3072] (tiled), K split over the "
                                 "waves of one workgroup, + bias + GELU",
                       "kernel_ms": aup_ms, "achieved_gbs": aup_bytes / (aup_ms * 1e-3) / 1e9,
                       "frac_hbm": aup_bytes / (aup_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, "algorithmic_bytes": aup_bytes,
                       "traffic": measured_traffic("gemm_skinny_ffn_up")}}

    # CPU baseline: the oracle's algorithm through its fp32 CPU port
    # (oracle/cpu_port.c: blocked AVX2-FMA products and vectorised attention,
    # OpenMP) on the first LS layers at full width (prompt K/V, prefix
    # layers, SS denoise steps over those layers), scaled by layers and steps.
    import oracle
    L, S = cfg["n_layers"], cfg["num_steps"]
    LS, SS = min(4, L), min(2, S)
    first = tuple(f"gwp.blocks.{l}." for l in range(LS))
    w = _read_weights(be, m, lambda n: not n.startswith("gwp.blocks.") or n.startswith(first)
                      or "scale_shift_table" in n)
    lib.wamx_gwp_free(m)
    oracle.set_port(True)
    ref = oracle.Gwp(cfg, w)
    t0 = time.perf_counter()
    ref.prompt(prompt, layers=LS)
    t1 = time.perf_counter()
    ref.prefix(state, latent, prompt, layers=LS)
    t2 = time.perf_counter()
    ref.denoise(noise, layers=LS, steps=SS)
    t3 = time.perf_counter()
    ref.close()
    oracle.set_port(False)
    cpu_ms = (t2 - t0) * 1e3 * L / LS + (t3 - t2) * 1e3 * (L * S) / (LS * SS)
    cores, model = cpu_info()
    cpu = {"value": cpu_ms, "unit": "ms per action chunk", "cores": oracle.num_threads(), "kind": "port",
           "sample": f"the oracle's algorithm through its fp32 CPU port (oracle/cpu_port.c: bf16 operands, fp32 "
                     f"accumulation, cache-blocked AVX2-FMA products, vectorised attention, OpenMP; -O3 "
                     f"-march=x86-64-v3): the first {LS} layers (prompt K/V + prefix layers + {SS} denoise steps "
                     f"over them, {(t3 - t0):.1f} s), scaled x{L / LS:g} (prompt, prefix) and x{L * S / (LS * SS):g} "
                     f"(denoise), on {model} ({cores} logical CPUs)"}
    return {"metric": "ms per action chunk (GWP-0.5-shape MoT, bf16, 1 GPU); GEMM % of MFMA peak", "unit": "ms",
            "value": ms, "ms_per_step": ms, "higher_is_better": False, "dtype": "bf16",
            "config": {"workload": "GWP-0.5-shaped MoT action chunk: 30 layers, d=3072, 24x128 heads, FFN 14336, "
                                   "prefix 1 state + 3x1024 visual tokens, 512 prompt tokens, 10 denoise steps on "
                                   "a 48x32 action chunk, batch 1",
                       "params": params, "graph_nodes": nodes,
                       "phase_ms": {"prompt": phases[0], "prefix": phases[1], "denoise": phases[2]},
                       "ms_per_chunk_back_to_back": ms_pipelined,
                       "ms_per_request_with_upload": ms_with_upload, "upload_bytes_per_request": upload_bytes,
                       "prompt_projection": "every request (wam-bench --mode raw)",
                       "ms_per_request_steady_prompt_cache": ms_steady,
                       "gemm_mfma_frac": roof["frac"]},
            "roofline": roof, "cpu_baseline": cpu}


def workload_decode(be, args):
    """The action-expert decode against a cached prefix: prompt and prefix
    caches of B chunks are filled once (untimed), then the 10-step unrolled
    denoise graph runs on them.  One step reads every action-expert weight
    once (289 MB per layer) and each chunk's KV (37.8 MB prefix + 6.3 MB
    prompt per layer); the GEMMs do 2 * 48B * sum(M*K) flops."""
    import ctypes as C
    lib = be.lib
    B = args.batch
    c = lib.wamx_gwp_default_config()
    c.batch = B
    cfg = {k: getattr(c, k) for k, _ in wamx.GwpConfig._fields_}
    m = lib.wamx_gwp_create(be.ptr, C.byref(c))
    if not m:
        raise RuntimeError(wamx.last_error())
    wamx.check(lib.wamx_gwp_init_synthetic(m, 0x5EED0004, 0.02), "init_synthetic")
    per = [_gwp_inputs(cfg, 0x5EED0004 + 17 * b) for b in range(B)]
    ins = [np.ascontiguousarray(np.concatenate([p[i] for p in per])) for i in range(4)]
    wamx.check(lib.wamx_gwp_set_inputs(m, *[a.ctypes.data for a in ins]), "set_inputs")
    wamx.check(lib.wamx_gwp_run_prompt(m), "prompt")
    wamx.check(lib.wamx_gwp_run_prefix(m), "prefix")
    for _ in range(max(1, args.warmup)):
        wamx.check(lib.wamx_gwp_run_denoise(m), "denoise")
    be.sync()
    t = wamx.Timer(be)
    t.start()
    for _ in range(args.steps):
        wamx.check(lib.wamx_gwp_run_denoise(m), "denoise")
    ms = t.stop_ms() / args.steps
    action = np.empty(B * cfg["action_chunk"] * cfg["action_dim"], np.float32)
    wamx.check(lib.wamx_gwp_get_action(m, action.ctypes.data), "get_action")
    if not np.all(np.isfinite(action)):
        raise RuntimeError("non-finite action chunk")
    L, S, T = cfg["n_layers"], cfg["num_steps"], cfg["action_chunk"]
    d, da, F, NL = cfg["hidden"], cfg["action_hidden"], cfg["action_ffn_dim"], cfg["n_lang"]
    P = 1 + cfg["grid_h"] * cfg["grid_w"]
    mk = 3 * d * da + da * d + d * da + da * d + 2 * F * da          # weight elements per layer
    kv = 2 * (P + NL) * d * 2                                          # K + V bytes per chunk and layer
    step_bytes = L * (2 * mk + B * kv)
    step_flops = L * (2 * B * T * mk + 4 * B * T * (P + T + NL) * d)
    gbs = step_bytes * S / (ms * 1e-3) / 1e9
    nodes = int(lib.wamx_gwp_graph_nodes(m, 2))
    lib.wamx_gwp_free(m)
    roof = {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
            "traffic": None, "kernel": f"denoise graph, {B} chunk(s): {L} layers x {S} steps",
            "bytes_per_step": step_bytes, "flops_per_step": step_flops,
            "tflops": step_flops * S / (ms * 1e-3) / 1e12}
    return {"metric": f"ms per decode of {B} action chunk(s) against a cached prefix (GWP-0.5-shape action "
                      f"expert, bf16, 1 GPU)", "unit": "ms", "value": ms, "ms_per_step": ms,
            "higher_is_better": False, "dtype": "bf16",
            "config": {"workload": f"action-expert decode, batch {B}: 10 denoise steps, 48 queries per chunk over "
                                   f"1+3072 self-attention and 512 prompt keys per layer, 30 layers, d=3072, 24x128, "
                                   f"FFN 14336", "batch": B, "ms_per_chunk": ms / B,
                       "chunks_per_s": B / (ms * 1e-3), "graph_nodes": nodes},
            "roofline": roof,
            "cpu_baseline": {"value": None, "unit": "ms", "cores": 0, "kind": "port",
                             "sample": "not run for this workload (the chunk workload reports the CPU baseline)"}}


WORKLOADS = {"chunk": workload_chunk, "ffn": workload_ffn, "gemm": workload_gemm, "decode": workload_decode}


def probe_traffic(be, launches: int = 3):
    """Launches for the rocprofv3 FETCH_SIZE / WRITE_SIZE passes: a streaming
    kernel of known size (bias_gelu_bf16 over 64 Mi bf16 values: 128 MiB read,
    128 MiB written) to scale the counters, then the roofline kernels at their
    chunk shapes.  Prints the algorithmic bytes of each as one JSON line."""
    lib = be.lib
    n, width = 64 << 20, 14336
    cx, cb, cy = be.array(_normal(n, 11, bf16=True)), be.array(_normal(width, 12, 0.0, 0.02, bf16=True)), be.empty(2 * n)
    for _ in range(launches):
        wamx.check(lib.wamx_op_bias_gelu_bf16(be.ptr, cx.ptr, cb.ptr, cy.ptr, n, width), "bias_gelu")
    be.sync()
    out = {"calibration": {"kernel": "bias_gelu_bf16_kernel", "read_bytes": 2 * n + 2 * width, "write_bytes": 2 * n}}
    D, F = 3072, 14336
    hw = _normal(F * D, 13, 0.0, 0.02, bf16=True)
    for key, T in (("gemm_dma_ffn_up", 3072), ("gemm_skinny_ffn_up", 48)):
        b = be.array(_normal(F, 14, 0.0, 0.02, bf16=True))
        x = be.array(_normal(T * D, 15, bf16=True))
        y = be.empty(T * F * 2)
        if T > 64:   # row-major weight, many-token GEMM
            w = be.array(hw)
            for _ in range(launches):
                wamx.check(lib.wamx_op_linear(be.ptr, w.ptr, x.ptr, wamx.TYPE_BF16, b.ptr, wamx.EPI_BIAS_GELU, None,
                                              None, y.ptr, F, T, D), "linear")
        else:        # the action expert's weights live in the tiled buffer type
            ctx = lib.wamx_init(4)
            wt = lib.wamx_new_tensor_2d(ctx, wamx.TYPE_BF16, D, F)
            buf = lib.wamx_backend_alloc_ctx_tensors_from_buft(ctx, lib.wamx_backend_tiled_buffer_type(0))
            if not buf:
                raise RuntimeError(wamx.last_error())
            wamx.check(lib.wamx_backend_tensor_set(wt, hw.ctypes.data, 0, hw.nbytes), "tensor_set")
            for _ in range(launches):
                wamx.check(lib.wamx_op_linear_tiled(be.ptr, wt.contents.data, x.ptr, wamx.TYPE_BF16, b.ptr,
                                                    wamx.EPI_BIAS_GELU, None, None, y.ptr, F, T, D), "linear_tiled")
        be.sync()
        out[key] = {"tokens": T, "read_bytes": F * D * 2 + T * D * 2 + F * 2, "write_bytes": T * F * 2}
        for a in (b, x, y):
            a.free()
        if T > 64:
            w.free()
        else:
            lib.wamx_buffer_free(buf)
            lib.wamx_free(ctx)
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="chunk", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=1, help="independent chunks (decode workload)")
    ap.add_argument("--probe-traffic", action="store_true",
                    help="only launch the counter-calibration and roofline kernels (for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by heads / independent chunks, see the design notes)", file=sys.stderr)
        sys.exit(2)
    be = wamx.Backend(0)
    if args.probe_traffic:
        probe_traffic(be)
        be.close()
        return
    res = WORKLOADS[args.workload](be, args)
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": res["higher_is_better"],
            "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"], "data": "synthetic",
            "config": res["config"], "roofline": res["roofline"], "cpu_baseline": res["cpu_baseline"]}
    print(json.dumps(line), flush=True)
    be.close()


if __name__ == "__main__":
    main()
