#!/usr/bin/env python3
"""MM-DiT flow-step benchmark on one MI355X.

Workload (the configuration the metric is quoted on): one full MM-DiT flow
step at 9 s -- 194 latent tokens + 77 text tokens, CFG batch 2, d = 1024,
16 heads x 64, GELU(tanh) MLP 4x, 7 joint + 14 fused blocks, BF16 weights
random-init N(0, 0.02) from seed 1234, latent/text N(0, 1) from seed 4242,
t = 0.5. Inputs are resident in HBM before the timed region.

Prints ONE JSON line: steps/s (value), the roofline of the dominant kernel
class (measured with HIP events around its launches inside the timed steps),
attention TFLOP/s at 9 s and 30 s, the reference graph's SwiGLU conv MLP and
k3 convolution at 30 s, the Q8_0 projection GEMMs at 30 s, the 24-layer T5
encoder stack, and the CPU baseline (the oracle's restatement of the
same flow step on this host's cores).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0       # MI355X dense int8 MFMA
PEAK_FP32_TFLOPS = 157.3      # MI355X dense fp32 MFMA


def make_inputs(B, T, seed=4242):
    import numpy as np
    rng = np.random.default_rng(seed)
    lat = rng.standard_normal((B, T, 64), dtype=np.float32)
    txt = rng.standard_normal((B, 77, 1024), dtype=np.float32)   # row 0 cond, row 1 uncond
    return lat, np.full(B, 0.5, np.float32), txt


def roofline(role, ms, launches, flop, nbytes):
    """achieved rate of one launch class against the MI355X roof that bounds it."""
    if launches == 0 or ms <= 0:
        return None
    avg_s = ms / 1e3 / launches
    ai = flop / max(nbytes, 1.0)
    ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    if ai >= ridge:
        ach = flop / launches / avg_s / 1e12
        return {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": None,
                "kernel": role, "launches_per_step": None, "avg_us": round(avg_s * 1e6, 3),
                "flop_per_launch": flop / launches, "bytes_per_launch": nbytes / launches}
    ach = nbytes / launches / avg_s / 1e9
    return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None, "kernel": role,
            "launches_per_step": None, "avg_us": round(avg_s * 1e6, 3),
            "flop_per_launch": flop / launches, "bytes_per_launch": nbytes / launches}


def measured_traffic(role):
    """HBM bytes per launch of `role` at 9 s from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/hbm_traffic_flow_step_9s.md, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_flow_step_9s.md")
    try:
        lines = open(path).read().split("traffic_bytes_per_launch_9s", 1)[1].split("```")[0].split()
    except (OSError, IndexError):
        return None
    table = dict(zip(lines[0::2], lines[1::2]))
    return float(table[role]) if role in table else None


def cpu_info():
    """CPU model, the vector-ISA flags that matter to a GEMM, and core counts of this host."""
    model, flags = None, []
    try:
        for line in open("/proc/cpuinfo"):
            if model is None and line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
            if not flags and line.startswith("flags"):
                have = set(line.split(":", 1)[1].split())
                flags = [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512_vnni", "avx512_bf16",
                                     "amx_bf16", "amx_int8") if f in have]
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count() or 1
    return {"model": model, "flags": flags, "logical_cpus": os.cpu_count(), "allowed_cpus": allowed}


def cpu_baseline(weights, lat, t, txt, inputs30, runs=5, runs30=3):
    """The oracle's flow step (the same weights and inputs as the GPU step) on
    this host: one warm-up, then the median of `runs` timed steps, at 4
    threads (ggml-cpu's default thread count: the reference never sets
    n_threads, src/common/ts_backend.h:10-16) and at every allowed core (at
    most 16, the host share of one GPU); CFG as one B = 2 forward, and as the
    reference's two B = 1 forwards per step (src/mmdit.cpp:363-364) on all
    allowed cores. At 30 s (646 + 77 tokens, the sampler's step) the median
    of `runs30` steps at both thread counts (one warm-up on all cores), and
    the 24-step sample as 24 of those steps (each step runs the same
    forward; the CFG / Euler update is negligible next to it)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    info = cpu_info()
    nthreads = max(1, min(16, info["allowed_cpus"]))
    od = oracle.OracleDiT(oracle.dit_config())
    for k, v in weights.items():
        od.set_tensor(k, v)

    def timed(threads, fn):
        oracle.set_threads(threads)
        fn()
        walls = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            walls.append(time.perf_counter() - t0)
        return sorted(walls)[len(walls) // 2], [round(w, 3) for w in walls]

    b2 = lambda: od.forward(lat, t, txt, act_bf16=True, kv_f16=True)

    def two_b1():
        od.forward(lat[:1], t[:1], txt[:1], act_bf16=True, kv_f16=True)
        od.forward(lat[1:], t[1:], txt[1:], act_bf16=True, kv_f16=True)

    med_all, walls_all = timed(nthreads, b2)
    med_b1, walls_b1 = timed(nthreads, two_b1)
    med_4, walls_4 = timed(4, b2)
    lat30, t30, txt30 = inputs30
    b2_30 = lambda: od.forward(lat30, t30, txt30, act_bf16=True, kv_f16=True)
    oracle.set_threads(nthreads)
    b2_30()
    walls30 = {}
    for th in (nthreads, 4):
        oracle.set_threads(th)
        w = []
        for _ in range(runs30):
            t0 = time.perf_counter()
            b2_30()
            w.append(time.perf_counter() - t0)
        walls30[th] = (sorted(w)[len(w) // 2], [round(x, 3) for x in w])
    med30 = walls30[nthreads][0]
    step30 = {"threads": nthreads, "steps_per_s": round(1.0 / med30, 4), "median_s": round(med30, 4),
              "runs_s": walls30[nthreads][1],
              "threads_4": {"steps_per_s": round(1.0 / walls30[4][0], 4), "median_s": round(walls30[4][0], 4),
                            "runs_s": walls30[4][1]},
              "sample_24_steps_s": round(24 * med30, 2),
              "sample_24_steps_s_threads_4": round(24 * walls30[4][0], 2)}
    return {"value": round(1.0 / med_all, 4), "unit": "steps/s", "cores": nthreads, "kind": "port",
            "sample": f"one full 21-block CFG-batched flow step at 9 s (B=2, 194+77 tokens), the oracle's C "
                      f"restatement of ggml-cpu semantics on {nthreads} threads; 1 warm-up, median of {runs}",
            "cpu": info,
            "median_s": round(med_all, 4), "runs_s": walls_all,
            "threads_4": {"steps_per_s": round(1.0 / med_4, 4), "median_s": round(med_4, 4), "runs_s": walls_4},
            "cfg_two_b1_forwards": {"threads": nthreads, "steps_per_s": round(1.0 / med_b1, 4),
                                    "median_s": round(med_b1, 4), "runs_s": walls_b1},
            "step_30s": step30}


def conv_bench(tsk, reps=20, B=2, S=646, H=1024, F=2816, seed=77):
    """convmlp and conv_cl (src/mmdit.cpp:28-44) on device-resident operands:
    us per call (HIP events around `reps` back-to-back calls) and TFLOP/s."""
    import numpy as np
    rng = np.random.default_rng(seed)

    def kernel(oc, ic):
        w = (rng.standard_normal((oc, ic, 3)) * 0.02).astype(np.float32)
        u = w.view(np.uint32)
        bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)   # RNE to bf16
        return tsk.conv1d_pack_weight(tsk.bf16_to_device(bits))

    w1, w3, w2, wl = kernel(F, H), kernel(F, H), kernel(H, F), kernel(H, H)
    x = tsk.to_device(rng.standard_normal((B, S, H)).astype(np.float32))
    y = tsk.empty((B, S, H))
    out = {}
    for name, fn, flop in (
            ("conv_mlp_swiglu", lambda: tsk.conv_mlp_swiglu(w1, w3, w2, x, out=y), 3 * 2.0 * B * S * 3 * H * F),
            ("conv1d_linear1", lambda: tsk.conv1d(wl, x, out=y), 2.0 * B * S * 3 * H * H)):
        for _ in range(3):
            fn()
        tsk.synchronize()
        s, e = tsk.Event(), tsk.Event()
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        tsk.synchronize()
        us = s.elapsed_ms(e) / reps * 1e3
        tf = flop / (us * 1e-6) / 1e12
        out[name] = {"us": round(us, 2), "tflops": round(tf, 1), "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                     "shape": f"B={B} S={S} {H}->{F}->{H} k3" if name == "conv_mlp_swiglu" else f"B={B} S={S} {H}->{H} k3"}
    return out


def attention_node_bench(tsk, reps=20, B=2, H=16, N=723, seed=33, types="ref"):
    """The flash_attn_ext node at the 30 s joint attention (646 latent + 77
    text tokens, 16 x 64 heads, B = 2; scale 1/8, F32 precision, f32 output) on
    device-resident N(0, 1) operands (what QK-RMSNorm leaves: rows of unit
    RMS). types "ref": the node mmdit.cpp:88-92 emits, Q F32 with K / V cast
    to F16 (V read as rows by the kernel, one launch); "bf16": bf16 Q / K / V
    (V transposed to fp16 first, two launches). The C entry point is called
    with prebuilt descriptors, so the Python wrapper's own cost stays out of
    the loop. us per call and TFLOP/s by 4 B H N^2 64."""
    import ctypes
    import numpy as np
    rng = np.random.default_rng(seed)

    def bf16(shape):
        u = rng.standard_normal(shape, dtype=np.float32).view(np.uint32)
        return tsk.bf16_to_device(((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16))

    if types == "ref":
        f = lambda: rng.standard_normal((B, H, N, 64), dtype=np.float32)
        q, k, v = tsk.to_device(f()), tsk.to_device(f().astype(np.float16)), tsk.to_device(f().astype(np.float16))
    else:
        q, k, v = bf16((B, H, N, 64)), bf16((B, H, N, 64)), bf16((B, H, N, 64))
    out = tsk.empty((B, N, H, 64))
    tsk.init()
    L = tsk.load()
    dq, dk, dv, dd = tsk.desc(q), tsk.desc(k), tsk.desc(v), tsk.desc(out)
    st = tsk._stream()
    args = (ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv), None, 0.125, 0.0, 0.0, tsk.PREC_F32,
            ctypes.byref(dd), st)
    for _ in range(3):
        tsk.check(L.tsk_flash_attn_ext(*args))
    tsk.synchronize()
    s, e = tsk.Event(), tsk.Event()
    s.record()
    bad = 0
    for _ in range(reps):
        bad |= L.tsk_flash_attn_ext(*args)
    e.record()
    tsk.synchronize()
    tsk.check(bad)
    us = s.elapsed_ms(e) / reps * 1e3
    tf = 4.0 * B * H * N * N * 64 / (us * 1e-6) / 1e12
    shape = ("Q F32, K / V F16 (mmdit.cpp:88-90)" if types == "ref" else "bf16 Q / K / V")
    return {"us": round(us, 2), "tflops": round(tf, 1), "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "shape": f"B={B} H={H} N={N} D=64, {shape}, f32 output",
            "launches": 1 if types == "ref" else 2}


def q8_blocks(rng, M, K, scale):
    """ggml Q8_0 blocks (M, K/32, 34) uint8: fp16 scale then int8 values uniform in [-127, 127]."""
    import numpy as np
    qs = rng.integers(-127, 128, size=(M, K // 32, 32), dtype=np.int8)
    d = np.full((M, K // 32, 1), np.float16(scale)).view(np.uint8)
    return np.ascontiguousarray(np.concatenate([d.reshape(M, K // 32, 2), qs.view(np.uint8)], axis=2))


def q8_bench(tsk, reps=10, N=1446, seed=5):
    """The four Q8_0 projection GEMMs at 30 s (2 x 723 rows), weights repacked
    once, activations quantized per call (ggml's conversion of src1)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    rows, tot_us, tot_ops = {}, 0.0, 0.0
    for K, M in ((1024, 3072), (1024, 1024), (1024, 4096), (4096, 1024)):
        w = tsk.q8_0_repack(tsk.to_device(q8_blocks(rng, M, K, 1.0 / (127.0 * np.sqrt(K)))))
        x = tsk.to_device(rng.standard_normal((N, K)).astype(np.float32))
        y = tsk.empty((N, M))
        fn = lambda: tsk.mul_mat(w, x, out=y, a_type=tsk.Q8_0_SPLIT)
        for _ in range(3):
            fn()
        tsk.synchronize()
        s, e = tsk.Event(), tsk.Event()
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        tsk.synchronize()
        us = s.elapsed_ms(e) / reps * 1e3
        ops = 2.0 * N * K * M
        rows[f"{K}->{M}"] = {"us": round(us, 2), "tops": round(ops / us / 1e6, 1)}
        tot_us += us
        tot_ops += ops
    return {"rows": N, "gemms": rows, "total_us": round(tot_us, 2), "tops": round(tot_ops / tot_us / 1e6, 1),
            "frac_of_int8_peak": round(tot_ops / tot_us / 1e6 / PEAK_INT8_TOPS, 4)}


def t5_bench(tsk, seed=44, reps=3):
    """Configuration 4: the 24-layer T5 encoder stack on 512 tokens (last 64
    padded), random Q8_0 weights; wall time of one encode with the operands
    resident (median of reps)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    t5 = tsk.T5(tsk.t5_config())
    for name, ne, ty in t5.tensors():
        if ty == 8:
            s = 1.0 / np.sqrt(ne[0] * 127.0 * 127.0 / 3.0)
            if name.endswith(".q") or name.endswith(".k"):
                s /= np.sqrt(8.0)
            t5.set_tensor(name, q8_blocks(rng, ne[1], ne[0], s))
        elif name == "rel_bias":
            t5.set_tensor(name, rng.standard_normal((ne[1], ne[0])).astype(np.float32))
        else:
            t5.set_tensor(name, (1.0 + 0.1 * rng.standard_normal(ne[0])).astype(np.float32))
    c = t5.cfg
    x = tsk.to_device(rng.standard_normal((512, c.d_model)).astype(np.float32))
    ids = np.arange(1, 513, dtype=np.int32)
    ids[-64:] = 0
    out = tsk.empty((512, c.d_model))
    t5.encode_device(x, ids, out)
    tsk.synchronize()
    walls = []
    for _ in range(reps):
        t0 = time.perf_counter()
        t5.encode_device(x, ids, out)
        tsk.synchronize()
        walls.append(time.perf_counter() - t0)
    wall = sorted(walls)[len(walls) // 2]
    per_layer = 2.0 * 512 * c.d_model * (3 * c.n_heads * c.d_kv + c.n_heads * c.d_kv + 2 * c.d_ff) + \
        2.0 * 512 * c.d_ff * c.d_model + 4.0 * c.n_heads * 512 * 512 * c.d_kv
    t5.close()
    return {"layers": c.n_layers, "tokens": 512, "ms": round(wall * 1e3, 3),
            "tops": round(per_layer * c.n_layers / wall / 1e12, 1)}


def graph_bench(tsk, steps, warmup=3):
    """the reference's own MM-DiT graph (tsk_mmdit: latent | clip | text
    streams, k3 conv linear1 / convMLP, SwiGLU MLPs of 2816, per-token
    extended_c adaLN, 154 text tokens, k7 output conv; src/mmdit.cpp:119-342)
    at 9 s (194 latent, 72 clip, 216 sync frames) and 30 s (646, 240, 720):
    one B = 2 (CFG) forward per step, inputs resident in HBM, HIP events around
    `steps` forwards; the 24-step CFG-5 sampler at 30 s (wall clock, host
    inputs and result); and the same graph with the Q8_0 GGUF's weight types
    (convert/quantize_gguf.py: 2-D linears Q8_0, the 3-D convolution kernels
    F32, their products as three bf16 ones each: the library's default)"""
    import numpy as np
    out = {}
    rng = np.random.default_rng(4242)
    shapes = (("9s", 194, 72, 216), ("30s", 646, 240, 720))
    inputs = {}
    for label, T, Sc, Ss in shapes:
        f = lambda *sh: rng.standard_normal(sh, dtype=np.float32)
        inputs[label] = (f(2, 64, T), f(2, Sc, 1024), f(2, Ss, 768), f(2, 77, 1024), f(2, 77, 2048), f(2, 1024))

    def timed_forwards(m, label, T, Sc, Ss, n, nwarm):
        host = inputs[label]
        dev = [tsk.to_device(a) for a in host]
        t = np.full(2, 0.5, np.float32)
        flow = tsk.empty((2, T, 64))
        for _ in range(nwarm):
            m.forward_device(dev[0], t, *dev[1:], flow)
        tsk.synchronize()
        s, e = tsk.Event(), tsk.Event()
        s.record()
        for _ in range(n):
            m.forward_device(dev[0], t, *dev[1:], flow)
        e.record()
        tsk.synchronize()
        ms = s.elapsed_ms(e) / n
        return {"steps_per_s": round(1000.0 / ms, 2), "ms_per_step": round(ms, 4), "latent_tokens": T,
                "clip_frames": Sc, "sync_frames": Ss, "joint_tokens": T + Sc + 154}

    m = tsk.MMDit(tsk.mmdit_config())
    for k, v in tsk.mmdit_pool_weights(m.tensors()):
        m.set_tensor(k, v)
    for label, T, Sc, Ss in shapes:
        out[label] = timed_forwards(m, label, T, Sc, Ss, steps, warmup)
    host = inputs["30s"]
    a = (host[0][0], host[1][0], host[2][0], host[3][0], host[4][0], host[5][0])
    m.sample(*a, steps=24, cfg_scale=5.0)
    walls = []
    for _ in range(3):
        t0 = time.perf_counter()
        m.sample(*a, steps=24, cfg_scale=5.0)
        walls.append(time.perf_counter() - t0)
    wall = sorted(walls)[1]
    out["sample_24_steps_30s"] = {
        "seconds": round(wall, 4), "sampler_steps_per_s": round(24 / wall, 2),
        "vs_24_forwards": round(wall / (24 * out["30s"]["ms_per_step"] / 1e3), 4),
        "note": "t-independent conditioning once per sample, latent and CFG / Euler on the device; "
                "wall clock incl. the host inputs' upload and the result's download"}
    m.close()
    out["weights"] = "BF16 (t_embed MLP F32), 1.28 G parameters, random-init from a seeded N(0, 0.02) pool"
    mq = tsk.MMDit(tsk.mmdit_config(weight_type=8))
    for k, v in tsk.mmdit_pool_weights(mq.tensors()):
        mq.set_tensor(k, v)
    out["q8_0"] = {label: timed_forwards(mq, label, T, Sc, Ss, max(3, steps // 2), 1) for label, T, Sc, Ss in shapes}
    out["q8_0"]["weights"] = ("the Q8_0 GGUF's types: 2-D linears Q8_0 (ggml's reference quantizer), 3-D "
                              "convolution kernels, t_embed MLP and vectors F32")
    out["q8_0"]["f32_products"] = ("F32 convolution kernels as three bf16 products (weight planes [hi | lo | hi] "
                                   "against activation planes [hi | hi | lo], ~2^-17 of |x w| per term); "
                                   "TSK_F32_SPLIT=0 runs them on fp32 MFMA")
    mq.close()
    return out


def vae_bench(tsk, reps=3):
    """the Oobleck VAE decode of a 9 s (194 latent frames -> 397312 samples)
    and a 30 s (646 -> 1323008) latent, F32 weights (random, variance
    preserving), latent resident in HBM; HIP events around `reps` decodes"""
    import numpy as np
    v = tsk.Vae(tsk.vae_config(max_latent=646))
    weights = tsk.vae_synthetic_weights(v.tensors(), seed=77, snake_std=0.1)
    for k, w in weights.items():
        v.set_tensor(k, w)
    out, ref_audio = {}, {}
    rng = np.random.default_rng(4242)
    for label, T in (("9s", 194), ("30s", 646)):
        lat = tsk.to_device(rng.standard_normal((64, T), dtype=np.float32))
        audio = tsk.empty((2, T * v.hop))
        v.decode_device(lat, audio)
        tsk.synchronize()
        s, e = tsk.Event(), tsk.Event()
        s.record()
        for _ in range(reps):
            v.decode_device(lat, audio)
        e.record()
        tsk.synchronize()
        ms = s.elapsed_ms(e) / reps
        fl = vae_flops(tsk.vae_config(), T)
        tf = fl / (ms / 1e3) / 1e12
        out[label] = {"ms": round(ms, 3), "latent_frames": T, "samples": T * v.hop,
                      "realtime_factor": round(T * v.hop / 44100.0 / (ms / 1e3), 1),
                      "tflops": round(tf, 1), "frac_of_fp32_peak": round(tf / PEAK_FP32_TFLOPS, 4)}
        ref_audio[label] = (lat, audio.numpy().astype(np.float64))
    # the opt-in split products (TSK_VAE_SPLIT=1 at creation): the same decode
    # with every convolution but the output one as three bf16 products
    os.environ["TSK_VAE_SPLIT"] = "1"
    tsk.init(0, reread=True)
    try:
        vs = tsk.Vae(tsk.vae_config(max_latent=646))
        for k, w in weights.items():
            vs.set_tensor(k, w)
        split = {}
        for label, T in (("9s", 194), ("30s", 646)):
            lat, a64 = ref_audio[label]
            audio = tsk.empty((2, T * vs.hop))
            vs.decode_device(lat, audio)
            tsk.synchronize()
            s, e = tsk.Event(), tsk.Event()
            s.record()
            for _ in range(reps):
                vs.decode_device(lat, audio)
            e.record()
            tsk.synchronize()
            ms = s.elapsed_ms(e) / reps
            d = audio.numpy().astype(np.float64) - a64
            split[label] = {"ms": round(ms, 3), "realtime_factor": round(T * vs.hop / 44100.0 / (ms / 1e3), 1),
                            "rel_l2_vs_fp32_products": float(np.sqrt((d ** 2).sum() / (a64 ** 2).sum()))}
        split["note"] = ("TSK_VAE_SPLIT=1: F32 products as three bf16 products (weight planes [hi | lo | hi] x "
                         "input planes [hi | hi | lo]); the default decode above uses fp32 MFMA products")
        out["split_products"] = split
        vs.close()
    finally:
        os.environ.pop("TSK_VAE_SPLIT", None)
        tsk.init(0, reread=True)
    v.close()
    return out


def vae_flops(c, T):
    """Multiply-adds x 2 of the Oobleck decoder's convolutions for T latent
    frames (src/vae_decoder.cpp:62-124): conv k7 latent -> 16 C; per block
    (multipliers run backwards) a transposed convolution of stride s whose
    output samples each take 2 taps (kernel 2 s) and three residual units of a
    k7 and a k1 convolution; the final k7 conv C -> out. (The device runs
    each transposed convolution as two 2-tap phase products, the work counted
    here; the reference's zero-stuffed form does s x more.)"""
    C = c.channels
    mult = [1] + list(c.c_mults)
    t = T
    fl = 2.0 * t * mult[5] * C * c.latent_dim * 7
    for n in range(5):
        ic, oc, st = mult[5 - n] * C, mult[4 - n] * C, c.strides[4 - n]
        t *= st
        fl += 2.0 * t * oc * ic * 2 + 3 * 2.0 * t * oc * oc * (7 + 1)
    return fl + 2.0 * t * c.out_channels * C * 7


def copy_calibration(nbytes=256 << 20, reps=5):
    """A plain device-to-device copy of known size: each launch reads and writes nbytes."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": reps}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (the reference kernel of known "
                         "traffic that rocprofv3 FETCH_SIZE / WRITE_SIZE readings are scaled by)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs the MM-DiT step on one GPU "
              f"only (CFG/data sharding over several GPUs is a design note in DESIGN.md); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    from __graft_entry__ import ensure_built, load_tsk

    ensure_built()
    tsk = load_tsk()
    tsk.init(0)
    dit = tsk.Dit(tsk.dit_config(max_batch=2, max_latent=646))
    weights = tsk.synthetic_weights(dit.tensors(), seed=1234)
    for k, v in weights.items():
        dit.set_tensor(k, v)

    def run(T, steps, warmup, timing):
        lat, t, txt = make_inputs(2, T)
        # ts_dit::forward's latent layout ne = [T, 64, B]
        lat_d, txt_d = tsk.to_device(np.ascontiguousarray(lat.transpose(0, 2, 1))), tsk.to_device(txt)
        flow = tsk.empty((2, T, 64))
        for _ in range(warmup):
            dit.forward_device(lat_d, t, txt_d, flow)
        tsk.synchronize()
        if timing:
            dit.timing(True)
        s, e = tsk.Event(), tsk.Event()
        s.record()
        for _ in range(steps):
            dit.forward_device(lat_d, t, txt_d, flow)
        e.record()
        tsk.synchronize()
        ms = s.elapsed_ms(e) / steps
        roles = None
        if timing:
            dit.timing(False)
            roles = dit.timing_read()
        return ms, roles, (lat, t, txt)

    # config 2 (9 s): timed steps; per-kernel HIP events around every launch inside them
    ms_plain, _, inputs9 = run(194, args.steps, args.warmup, False)
    ms_timed, roles9, _ = run(194, args.steps, 1, True)
    # the host entry point tsk_dit_forward at 9 s: host latent / text in, flow
    # out, the PCIe copies and the final synchronisation inside the timing
    lat_h = np.ascontiguousarray(inputs9[0].transpose(0, 2, 1))
    dit.forward(lat_h, inputs9[1], inputs9[2])
    t_host = time.perf_counter()
    for _ in range(args.steps):
        dit.forward(lat_h, inputs9[1], inputs9[2])
    ms_host = (time.perf_counter() - t_host) * 1e3 / args.steps
    # 30 s (646 latent + 77 text tokens): steps/s (plain), attention at N = 723 (timed)
    ms30, _, inputs30 = run(646, max(5, args.steps // 2), 2, False)
    _, roles30, _ = run(646, max(5, args.steps // 2), 1, True)
    # the same 30 s step with every q / k RMSNorm weight scaled by 2.5: logits
    # beyond the bound of the max-free softmax, so every attention launch runs
    # the running-max kernel (trained norm weights may be that large)
    norms = {k: v for k, v in weights.items() if k.endswith("norm.weight")}
    for k, v in norms.items():
        dit.set_tensor(k, v * np.float32(2.5))
    ms30u, roles30u, _ = run(646, max(5, args.steps // 2), 2, True)
    for k, v in norms.items():
        dit.set_tensor(k, v)

    # config 5: the full 24-step rectified-flow Euler sampler with CFG 5 at 30 s
    # (646 latent + 77 text tokens, cond/uncond batched as B = 2 per step),
    # noise N(0, 1) from seed 4242; wall clock around tsk_dit_sample (one
    # warm-up sample, median of 3)
    rng = np.random.default_rng(4242)
    noise = np.ascontiguousarray(rng.standard_normal((646, 64), dtype=np.float32).T)   # ne = [T, 64]
    tc = rng.standard_normal((77, 1024), dtype=np.float32)
    tu = rng.standard_normal((77, 1024), dtype=np.float32)
    dit.sample(noise, tc, tu, steps=24, cfg_scale=5.0)
    walls = []
    for _ in range(3):
        t0 = time.perf_counter()
        dit.sample(noise, tc, tu, steps=24, cfg_scale=5.0)
        walls.append(time.perf_counter() - t0)
    wall = sorted(walls)[1]
    sample30 = {"steps": 24, "cfg_scale": 5.0, "latent_tokens": 646, "seconds": round(wall, 5),
                "sampler_steps_per_s": round(24 / wall, 2), "ms_per_step": round(wall / 24 * 1e3, 4)}

    # the Q8_0 driver (block projections as Q8_0 weights, Q8_0 x Q8_0 products)
    # on the 9 s step: the same seeded weights, quantized with ggml's reference
    # quantizer by tsk_dit_set_tensor
    dq = tsk.Dit(tsk.dit_config(max_batch=2, max_latent=194, weight_type=8))
    for k, v in weights.items():
        dq.set_tensor(k, v)
    lat, t, txt = make_inputs(2, 194)
    lat_d, txt_d = tsk.to_device(np.ascontiguousarray(lat.transpose(0, 2, 1))), tsk.to_device(txt)
    flow_q = tsk.empty((2, 194, 64))
    for _ in range(args.warmup):
        dq.forward_device(lat_d, t, txt_d, flow_q)
    tsk.synchronize()
    sq, eq = tsk.Event(), tsk.Event()
    sq.record()
    for _ in range(args.steps):
        dq.forward_device(lat_d, t, txt_d, flow_q)
    eq.record()
    tsk.synchronize()
    ms_q8 = sq.elapsed_ms(eq) / args.steps
    dq.timing(True)
    for _ in range(args.steps):
        dq.forward_device(lat_d, t, txt_d, flow_q)
    tsk.synchronize()
    dq.timing(False)
    roles_q8 = dq.timing_read()
    dq.close()

    # the reference graph's convolution glue at 30 s (B = 2, 646 positions):
    # convmlp 1024 -> 2816 -> 1024 (k3, padding 1, SwiGLU) and a conv_cl
    # linear1 1024 -> 1024 (k3), BF16 kernels packed kw-major once, f32 input
    conv30 = conv_bench(tsk, reps=max(5, args.steps))
    # configuration 3's attention as the ggml node (bf16 Q / K / V, 723 tokens)
    attn_node = attention_node_bench(tsk, reps=max(20, args.steps))
    attn_node_bf16 = attention_node_bench(tsk, reps=max(20, args.steps), types="bf16")
    # the reference's own three-stream graph at 9 s and 30 s
    graph = graph_bench(tsk, max(5, args.steps // 2))
    # the VAE decode after the sampler
    vae = vae_bench(tsk)
    # configuration 3's Q8_0 projection GEMMs at 30 s and configuration 4's T5 stack
    q8 = q8_bench(tsk)
    t5 = t5_bench(tsk)

    dom = max(roles9, key=lambda r: roles9[r][0])
    rf = roofline(dom, *roles9[dom])
    rf["launches_per_step"] = roles9[dom][1] // args.steps
    rf["traffic"] = measured_traffic(dom)

    def attn(roles, ms_steps):
        ms, n, fl, by = roles["attn"]
        tf = fl / (ms / 1e3) / 1e12
        return {"tflops": round(tf, 2), "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                "avg_us": round(ms * 1e3 / n, 3), "launches_per_step": n // ms_steps}

    def breakdown(roles, steps):
        return {r: {"ms_per_step": round(v[0] / steps, 4), "launches_per_step": v[1] // steps,
                    "tflops": round(v[2] / (v[0] / 1e3) / 1e12, 2) if v[0] > 0 else None}
                for r, v in roles.items()}
    out = {
        "metric": "DiT flow steps/s at 9 s (CFG b=2)",
        "value": round(1000.0 / ms_plain, 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_plain, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, random-init N(0,0.02) BF16 weights)",
        "config": {"workload": "MM-DiT flow step, 9 s: 194 latent + 77 text tokens, CFG batch 2, "
                               "d=1024, 16x64 heads, GELU MLP 4x, 7 joint + 14 fused blocks, BF16 weights",
                   "global_batch": 2, "seq_len": 271, "parallelism": "single GPU"},
        "roofline": rf,
        "attention": {"9s": attn(roles9, args.steps), "30s": attn(roles30, max(5, args.steps // 2)),
                      "30s_unbounded": dict(attn(roles30u, max(5, args.steps // 2)),
                                            step_ms=round(ms30u, 4),
                                            note="q / k norm weights x 2.5: the running-max kernel; step_ms "
                                                 "includes per-launch HIP events")},
        "steps_per_s_30s": round(1000.0 / ms30, 2),
        "sample_24_steps_30s": sample30,
        "ms_per_step_with_kernel_events": round(ms_timed, 4),
        "host_entry_9s": {"steps_per_s": round(1000.0 / ms_host, 2), "ms_per_step": round(ms_host, 4),
                          "note": "tsk_dit_forward from host buffers: PCIe copies in and out and a "
                                  "synchronisation per step included"},
        "breakdown_9s": breakdown(roles9, args.steps),
        "breakdown_30s": breakdown(roles30, max(5, args.steps // 2)),
        "conv_30s": conv30,
        "attention_node_30s": attn_node,
        "attention_node_bf16_30s": attn_node_bf16,
        "q8_0_projections_30s": q8,
        "q8_0_flow_step_9s": {"steps_per_s": round(1000.0 / ms_q8, 2), "ms_per_step": round(ms_q8, 4),
                              "weights": "Q8_0 attn.qkv / linear1 / ffn.fc1 / ffn.fc2 (ggml reference "
                                         "quantizer), other matrices BF16",
                              "breakdown": breakdown(roles_q8, args.steps)},
        "t5_encoder_config4": t5,
        "reference_graph": graph,
        "vae_decode": vae,
    }
    if not args.no_cpu_baseline:
        lat, t, txt = inputs9
        out["cpu_baseline"] = cpu_baseline(weights, lat, t, txt, inputs30)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
