"""Benchmark: ViT-B/16 q2 forward on one MI355X (images/s), with the roofline
of the packed complex-phase GEMM and the CPU oracle timed beside it.

    python bench.py [--steps K] [--warmup W] [--config vit_b16_q2] [--batch B]

One step = one forward pass of the configured model over one synthetic batch
already resident in HBM.  Prints ONE JSON line (see README of the contract):
value = images/s; roofline = the packed-layer kernel with the most time in
the timed region (every launch of it, timed with HIP events on its launch
stream; roofline.by_kernel gives each packed kernel's own figures);
cpu_baseline = the numpy oracle's GEMM-only restatement of the same layers on
a bounded sample, run on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rpfq-review_amd"))
sys.path.insert(0, ROOT)

METRIC = "images/sec ViT-B/16 q2 bs256 on 1 MI355X; cplx-GEMM % MFMA/HBM peak"
PEAK_F16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0

# config -> (model name, batch, image size, codebook, seed, description)
CONFIGS = {
    "vit_b16_q2": ("rpfq_vit_base_patch16_224_q", 256, 224, "axis", 2,
                   "ViT-B/16 q2: complex_phase_v2 2-bit codes (4 planes), per-(plane,row) scales ~U(0.01,0.1)"),
    "deit_ti_q2": ("rpfq_deit_tiny_patch16_224_q", 64, 224, "axis", 1,
                   "DeiT-Tiny/16 distilled q2, 198 tokens"),
    "swin_t_q2": ("rpfq_swin_tiny_patch4_window7_224_q", 128, 224, "axis", 3,
                  "Swin-T q2 (patch-merging reductions quantized)"),
    "vit_l16_psk16": ("rpfq_vit_large_patch16_224_q", 512, 224, "psk16", 4,
                      "ViT-L/16 16-PSK 4-bit phase codes (U, W single stage)"),
}


def build_model(cfg_name: str, act_quant: bool = False, dtype=None):
    import torch
    import quant_models as qm
    from quant_models import _native as N
    from quant_models.inference import load_synthetic_codes, prepare_inference

    name, _, img, codebook, seed, _ = CONFIGS[cfg_name]
    torch.manual_seed(seed)
    model = qm.create_model(name, img_size=img, quant_method_u="complex_phase_v2",
                            quant_method_w="complex_phase_v2", enable_act_quant=act_quant, enable_rotation=False)
    cb = N.CB_PSK16 if codebook == "psk16" else N.CB_AXIS
    load_synthetic_codes(model, seed, cb)
    prepare_inference(model, "cuda", dtype or torch.float16)
    return model


def rows_per_image(model, x):
    """Rows each packed layer sees per image in one forward (pre-hooks)."""
    import torch
    from quant_models.inference import quant_layers

    from quant_models import vision_transformer as vt

    rows, hooks = {}, []
    for name, layer in quant_layers(model):
        def hook(mod, inp, name=name):
            rows[name] = inp[0].numel() // inp[0].shape[-1] // x.shape[0]
        hooks.append(layer.register_forward_pre_hook(hook))
    fused, vt.FUSED_BLOCKS = vt.FUSED_BLOCKS, False  # module calls only, so every hook fires
    try:
        with torch.no_grad():
            model(x[:1].repeat(x.shape[0], 1, 1, 1) if x.shape[0] > 1 else x)
    finally:
        vt.FUSED_BLOCKS = fused
        for h in hooks:
            h.remove()
    return rows


def cpu_baseline(model, rows: dict, budget_s: float = 12.0):
    """GEMM-only restatement of the reference's packed layers (decoded A_q,
    float32 numpy BLAS) over the model's quantized linears for whole images,
    repeated until `budget_s` of host time; returns images/s."""
    import numpy as np
    from oracle import rpfq_oracle as O
    from quant_models.inference import quant_layers

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = len(os.sched_getaffinity(0))
    layers = []
    for name, layer in quant_layers(model):
        lc = layer._override
        planes = []
        kinds = ["u"] * (len(lc.planes) // 2) + ["w"] * (len(lc.planes) // 2)
        for p, sre, sim, kind in zip(lc.planes, lc.scale_re, lc.scale_im, kinds):
            p = p.cpu().numpy()
            codes = O.unpack_codes4(p) if lc.codebook == 2 else O.unpack_codes(p)
            planes.append((codes[:, :lc.k_complex], sre.cpu().numpy()[:, 0], sim.cpu().numpy()[:, 0], kind))
        a = O.wide_weight(planes, "psk16" if lc.codebook == 2 else "axis")
        layers.append((np.ascontiguousarray(a.T), rows[name]))
    rng = np.random.default_rng(0)
    xs = {}
    for a, r in layers:
        if xs.get(a.shape[0], np.empty((0, 0))).shape[0] < r:
            xs[a.shape[0]] = rng.standard_normal((r, a.shape[0])).astype(np.float32)
    ctx = threadpool_limits(limits=cores) if threadpool_limits else None
    if ctx:
        ctx.__enter__()
    try:
        images = 0
        t0 = time.perf_counter()
        while True:
            for a, rows in layers:
                _ = xs[a.shape[0]][:rows] @ a
            images += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        dt = time.perf_counter() - t0
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    return {"value": images / dt, "unit": "images/s", "cores": cores, "kind": "port",
            "sample": f"{images} image(s) x {len(layers)} packed layers, GEMM-only float32 numpy BLAS on "
                      f"decoded A_q (oracle/rpfq_oracle.py), {dt:.1f} s; excludes attention/LayerNorm"}


def config1_inputs(seed: int = 0):
    """X planes N(0,1) float32 [1576, 768]; 2-bit codes
    U{0..3} [3072, 768] packed low-bits-first [3072, 192]; per-output-channel
    scale s ~ U(0.01, 0.1) held as the exporter's fp16 gamma = fp16(1/s)
    (so the packed format carries it exactly), shared by re and im."""
    import numpy as np

    rng = np.random.default_rng(seed)
    m, k, n = 1576, 768, 3072
    xr = rng.standard_normal((m, k)).astype(np.float32)
    xi = rng.standard_normal((m, k)).astype(np.float32)
    codes = rng.integers(0, 4, size=(n, k), dtype=np.uint8)
    c = codes.reshape(n, k // 4, 4)
    packed = (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)
    s = rng.uniform(0.01, 0.1, size=(n, 1))
    gamma = (1.0 / s).astype(np.float16)
    return xr, xi, codes, packed, gamma


def config1_cpu_baseline(xr, xi, codes, gamma, budget_s: float = 12.0):
    """The reference's own CPU primitive on config 1: phaseLinearReference
    (RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:119-164, U-branch
    feed (xr, -xi), compiled from the reference sources into oracle/_ref),
    single-threaded as the reference runs it, on the first T tokens with T
    sized to ~budget_s from a short probe; TFLOP/s of the algorithmic 8 M K N.
    Falls back to the numpy oracle (oracle.phase_linear) without oracle/_ref."""
    import numpy as np
    from oracle import ref_lib

    k, n = xr.shape[1], codes.shape[0]
    lib = ref_lib.load()
    kind = "reference" if lib is not None else "port"

    def run(t):
        if lib is not None:
            return ref_lib.phase_linear(xr[:t], -xi[:t], codes, gamma, gamma, k)
        from oracle import rpfq_oracle as O
        inv = O.inv_gamma(gamma)[:, 0]
        return O.phase_linear(xr[:t], xi[:t], codes, inv, inv, conj_input=False)

    t0 = time.perf_counter()
    run(2)
    probe = max(time.perf_counter() - t0, 1e-4) / 2
    t = int(min(xr.shape[0], max(2, budget_s / probe)))
    t0 = time.perf_counter()
    run(t)
    dt = time.perf_counter() - t0
    return {"value": round(8.0 * t * k * n / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": kind,
            "sample": f"{t} of 1576 tokens x K={k} x N={n}, "
                      + ("phaseLinearReference (oracle/_ref, compiled from the reference's Android C++)"
                         if lib is not None else "numpy oracle.phase_linear") + f", {dt:.1f} s"}


def bench_config1(steps: int, warmup: int, cpu: bool, budget_s: float) -> int:
    """Config 1: one phase-quantized complex Linear at the ViT-B fc1 shape
    through rpfq_phase_linear (phase_linear_kernel: ternary fp16 MFMA
    operands, the float32 planes split into fp16 hi + lo terms, scales in
    the epilogue), U-branch semantics y = W x (conj_x = 0).  A step is one
    launch over the resident [1576, 768] planes; value = TFLOP/s of the
    algorithmic 8 M K N."""
    import ctypes

    import torch
    from quant_models import _native as N

    xr, xi, codes, packed, gamma = config1_inputs()
    m, k = xr.shape
    n = codes.shape[0]
    dev = torch.device("cuda")
    txr, txi = torch.from_numpy(xr).to(dev), torch.from_numpy(xi).to(dev)
    tcodes = torch.from_numpy(packed).to(dev)
    tg = torch.from_numpy(gamma).to(dev)
    yr = torch.empty(m, n, dtype=torch.float32, device=dev)
    yi = torch.empty_like(yr)
    lib = N.load()
    stream = torch.cuda.current_stream()

    def launch():
        N.check("rpfq_phase_linear", lib.rpfq_phase_linear(
            txr.data_ptr(), txi.data_ptr(), N.F32, 0, m, k, tcodes.data_ptr(), tg.data_ptr(), tg.data_ptr(), 0,
            n, yr.data_ptr(), yi.data_ptr(), N.F32, stream.cuda_stream or None))

    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = 8.0 * m * k * n
    nbytes = 8 * m * k + k * n // 4 + 4 * n + 8 * m * n
    tflops = flops / (ms / 1e3) / 1e12
    line = {
        "metric": "complex-GEMM TFLOP/s, config 1 (phase-quantized complex Linear 768->3072, M = 1576, "
                  "float32 planes, U-branch) on 1 MI355X",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 in/out (fp16 hi + lo MFMA operands, f32 accumulate)",
        "data": "synthetic (numpy default_rng(0): N(0,1) planes, uniform 2-bit codes, fp16 gammas of U(0.01, 0.1))",
        "config": {"workload": "cplx_fc1: BASELINE config 1, M=1576 (8 images x 197 tokens), K=768, N=3072 "
                               "complex, per-output-channel scales", "m": m, "k": k, "n": n},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_F16_TFLOPS, 4), "traffic": None,
                     "kernel": "rpfq::phase_linear_kernel<32, F32, F32, false> (one launch per step; float32 x "
                               "runs two fp16 MFMA passes, hi and lo, so the MFMA executes 2x the algorithmic "
                               "flops)",
                     "algorithmic_bytes": nbytes, "algorithmic_gbs": round(nbytes / (ms / 1e3) / 1e9, 1)},
        "cpu_baseline": config1_cpu_baseline(xr, xi, codes, gamma, budget_s) if cpu else None,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_as_is(model, rows: dict, batch: int, gemm_rate: float, act_bits: int, budget_s: float = 12.0):
    """Variant (i), the reference layer's per-call work as it is
    (QATLinearComplexPhase.forward, quant_i.py:513-554): every call
    requantizes the float32 master weight (oracle.quantized_weight: 2x2
    split, two residual axis stages for U and W, recombination), applies the
    activation quantization when the model has it (oracle.act_quant), then
    the float32 GEMM -- timed for one forward of B images (B = the bench
    batch, or fewer so it fits ~budget_s at the GEMM-only rate); images/s."""
    import numpy as np
    from oracle import rpfq_oracle as O
    from quant_models.inference import quant_layers

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = len(os.sched_getaffinity(0))
    b = int(max(1, min(batch, 0.5 * budget_s * gemm_rate)))
    rng = np.random.default_rng(1)
    layers = [(layer.weight.detach().float().cpu().numpy(), rows[name]) for name, layer in quant_layers(model)]
    xs = {}
    for w, r in layers:
        if xs.get(w.shape[1], np.empty((0, 0))).shape[0] < r * b:
            xs[w.shape[1]] = rng.standard_normal((r * b, w.shape[1])).astype(np.float32)
    ctx = threadpool_limits(limits=cores) if threadpool_limits else None
    if ctx:
        ctx.__enter__()
    try:
        t0 = time.perf_counter()
        for w, r in layers:
            a_q, _, _ = O.quantized_weight(w, "axis", 2, "axis", 2)
            x = xs[w.shape[1]][:r * b]
            if act_bits:
                h = x.shape[1] // 2
                x = np.concatenate(O.act_quant(x[:, :h], x[:, h:], act_bits), axis=1)
            _ = x @ a_q.T
        dt = time.perf_counter() - t0
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    return {"value": round(b / dt, 3), "unit": "images/s", "cores": cores, "kind": "port",
            "sample": f"one forward of {b} image(s) x {len(layers)} packed layers: per-call requantization of the "
                      f"float32 master weight + " + (f"{act_bits}-bit act quant + " if act_bits else "")
                      + f"float32 numpy GEMM (oracle/rpfq_oracle.py), {dt:.1f} s"}


# Complex layer shapes (K', N') of the ViT-B/16 and ViT-L/16 packed linears.
STREAM_SHAPES = {
    "vit_b.qkv": (384, 1152), "vit_b.proj": (384, 384), "vit_b.fc1": (384, 1536), "vit_b.fc2": (1536, 384),
    "vit_l.qkv": (512, 1536), "vit_l.proj": (512, 512), "vit_l.fc1": (512, 2048), "vit_l.fc2": (2048, 512),
}


def stream_layer(k_c: int, n_c: int, seed: int, copies: int = 1):
    """q2 (complex_phase_v2) layer of K' x N' with uniformly random axis codes
    and per-(plane, row) scales ~U(0.01, 0.1), packed by rpfq_wide_pack.
    copies > 1: one buffer of `copies` blobs of that layer, each with its own
    random code bytes (every byte is a valid (U, W) index pair), for a
    rotation over distinct weights.  Returns a list of PackedWide."""
    import torch
    from quant_models import _native as N
    from quant_models import ops

    g = torch.Generator(device="cuda").manual_seed(seed)
    planes = [torch.randint(0, 256, (n_c, k_c // 4), dtype=torch.uint8, device="cuda", generator=g)
              for _ in range(4)]
    sre = [torch.rand(n_c, 1, device="cuda", generator=g) * 0.09 + 0.01 for _ in range(4)]
    sim = [torch.rand(n_c, 1, device="cuda", generator=g) * 0.09 + 0.01 for _ in range(4)]
    pw = ops.PackedWide.from_planes(planes, sre, sim, n_c, k_c, N.CB_AXIS, 2, 0, None)
    del planes, sre, sim
    if copies == 1:
        return [pw]
    nb = pw.blob.numel()
    codes_bytes = ((-(-n_c // 32)) * (-(-k_c // 32)) * 1024 + 255) // 256 * 256
    big = torch.empty(copies, nb, dtype=torch.uint8, device="cuda")
    big.copy_(pw.blob.expand(copies, nb))
    big[:, :codes_bytes] = torch.randint(0, 256, (copies, codes_bytes), dtype=torch.uint8, device="cuda",
                                         generator=g)
    return [ops.PackedWide(n_c, k_c, N.CB_AXIS, 2, 0, big[i]) for i in range(copies)]


def stream_case(k_c: int, n_c: int, m: int, mode: str, gib: float, reps: int, seed: int = 5, dtype=None):
    """Batch-M weight streaming of one layer shape.
    mode "stacked": one launch with N' stacked to >= gib GiB of codes (the
    kernel's streaming rate at this K'); mode "rotate": >= gib GiB of distinct
    blobs of the real K' x N' layer, one launch each, replayed from a HIP
    graph (per-layer rate at batch M, launch gaps included).  Timed with HIP
    events on the launch stream; bytes are algorithmic (ops.wide_bytes)."""
    import torch
    from quant_models import ops

    dev = torch.device("cuda")
    if mode == "stacked":
        n_tot = -(-int(gib * (1 << 30)) // k_c)
        n_tot = -(-n_tot // 32) * 32
        layers = stream_layer(k_c, n_tot, seed)
    else:
        copies = -(-int(gib * (1 << 30)) // (k_c * n_c))
        layers = stream_layer(k_c, n_c, seed, copies)
    n_layer = layers[0].n_complex
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    dt = dtype or torch.float16
    from quant_models import _native as N
    # (KERNEL_GEMV: the persistent form wide_linear_gemv_persist_kernel at
    # 12 k-steps from 4096 tiles, whole 64-row groups and 16-bit y)
    kname = N.KERNEL_NAMES[layers[0].kernel_for(m, dt, dt)]
    x = torch.randn(m, 2 * k_c, device=dev, generator=g).to(dt)
    bias = torch.randn(2 * n_layer, device=dev, generator=g)
    y = torch.empty(m, 2 * n_layer, dtype=dt, device=dev)

    def run_all():
        for pw in layers:
            pw.linear_into(x, bias, y)

    run_all()  # warm up (kernel attributes, first-touch)
    torch.cuda.synchronize()
    ref = y.clone()
    graph = None
    if mode == "rotate":
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                run_all()
        torch.cuda.current_stream().wait_stream(s)
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(y, ref):
            raise AssertionError("graph replay differs from the eager launches")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        graph.replay() if graph is not None else run_all()
    e1.record()
    torch.cuda.synchronize()
    if not torch.equal(y, ref):
        raise AssertionError("timed launches differ from the warm-up result")
    ms = e0.elapsed_time(e1) / reps
    nbytes = len(layers) * ops.wide_bytes(m, n_layer, k_c)
    code_bytes = len(layers) * n_layer * k_c
    del layers
    torch.cuda.empty_cache()
    gbs = nbytes / (ms / 1e3) / 1e9
    launches = 1 if mode == "stacked" else int(code_bytes // (k_c * n_layer))
    # rotate: one small launch per real layer, so the figure is per-layer
    # latency (us_per_launch), not a streaming rate
    return {"k_complex": k_c, "n_complex": n_layer, "m": m, "mode": mode, "kernel": kname,
            "launches": launches, "code_gib": round(code_bytes / (1 << 30), 3),
            "us": round(ms * 1e3, 2), "us_per_launch": round(ms * 1e3 / launches, 2),
            "gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}


def stream_sweep(ms=(1, 4, 16), modes=("stacked", "rotate"), gib: float = 1.0, reps: int = 10, out=None,
                 shapes=None):
    rows = []
    for mode in modes:
        for name, (k_c, n_c) in STREAM_SHAPES.items():
            if shapes and name not in shapes:
                continue
            for m in ms:
                row = {"shape": name, **stream_case(k_c, n_c, m, mode, gib, reps)}
                rows.append(row)
                print(json.dumps(row), flush=True)
    if out:
        os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
        with open(out, "w") as f:
            json.dump(rows, f, indent=1)
    return rows


def layer_probe(n_c: int, k_c: int, m: int, steps: int, flags: int = 0) -> int:
    """One q2 layer of N' x K' (uniformly random code bytes, per-row scales)
    on m fp16 rows: `steps` launches of the packed kernel (the one `flags`
    select), timed with HIP events; prints one JSON line with the kernel,
    the time per launch and the algorithmic HBM rate (ops.wide_bytes)."""
    import torch
    from quant_models import ops

    pw = stream_layer(k_c, n_c, 1)[0]
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(m, 2 * k_c, device="cuda", generator=g).half()
    y = torch.empty(m, 2 * n_c, device="cuda", dtype=torch.float16)
    pw.linear_into(x, None, y, flags)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        pw.linear_into(x, None, y, flags)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / max(1, steps)
    flops = 2 * m * 2 * k_c * 2 * n_c
    gbs = ops.wide_bytes(m, n_c, k_c) / us / 1e3
    print(json.dumps({"layer_probe": [n_c, k_c], "m": m, "flags": flags,
                      "kernel": pw.kernel_for(m, torch.float16, torch.float16, flags), "launches": steps + 1,
                      "avg_us": round(us, 2), "tflops": round(flops / us / 1e6, 1), "gbs": round(gbs, 1),
                      "frac": round(gbs / PEAK_HBM_GBS, 4)}))
    return 0


GRAD_SHAPES = (("qkv", 1152, 384), ("proj", 384, 384), ("fc1", 1536, 384), ("fc2", 384, 1536))


def vs_library_bench(m: int, steps: int) -> int:
    """The forward of the ViT-B/16 q2 layer shapes at m rows (default bs256
    x 197 tokens): the packed kernel (rpfq_wide_linear, fp16 in and out,
    float32 bias) against the dense library GEMM on the same layer's decoded
    fp16 coefficients (F.linear with the bias, hipBLASLt), on the same box,
    alternating (packed, library) per shape; HIP events over `steps`
    calls each (both warmed first; medians of three alternations); fc1 also
    as the model runs it, with its GELU (fused into the packed store; torch's
    F.gelu after the library GEMM); prints one JSON line."""
    import torch
    import torch.nn.functional as F

    def timed(fn):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    rows = {}
    g = torch.Generator(device="cuda").manual_seed(5)
    for name, n_c, k_c in GRAD_SHAPES:
        pw = stream_layer(k_c, n_c, 1)[0]
        a16 = pw.decode(round_fp16=True).half()
        x = torch.randn(m, 2 * k_c, device="cuda", generator=g).half()
        bias = torch.randn(2 * n_c, device="cuda", generator=g) * 0.1
        b16 = bias.half()
        y = torch.empty(m, 2 * n_c, device="cuda", dtype=torch.float16)
        for _ in range(steps):  # warm clocks and caches for both before timing
            pw.linear_into(x, bias, y)
            F.linear(x, a16, b16)
        packed, dense = [], []
        for _ in range(3):
            packed.append(timed(lambda: pw.linear_into(x, bias, y)))
            dense.append(timed(lambda: F.linear(x, a16, b16)))
        us_p, us_d = sorted(packed)[1], sorted(dense)[1]  # medians of the three alternations
        flops = 2 * m * 2 * n_c * 2 * k_c
        row = {"n_complex": n_c, "k_complex": k_c, "packed_us": round(us_p, 1), "library_us": round(us_d, 1),
               "packed_tflops": round(flops / us_p / 1e6, 1), "library_tflops": round(flops / us_d / 1e6, 1)}
        rows[name] = row
        print(f"# vs library {name}: {row}", file=sys.stderr, flush=True)
        if name == "fc1":
            # as the model runs fc1: its GELU in the packed store against the
            # library GEMM followed by torch's GELU
            from quant_models import _native as N
            packed, dense = [], []
            for _ in range(3):
                packed.append(timed(lambda: pw.linear_into(x, bias, y, N.FLAG_GELU)))
                dense.append(timed(lambda: F.gelu(F.linear(x, a16, b16))))
            us_p, us_d = sorted(packed)[1], sorted(dense)[1]
            row = {"n_complex": n_c, "k_complex": k_c, "packed_us": round(us_p, 1), "library_us": round(us_d, 1)}
            rows["fc1+gelu"] = row
            print(f"# vs library fc1+gelu: {row}", file=sys.stderr, flush=True)
        del pw, a16, x, y
        torch.cuda.empty_cache()
    plain = ("qkv", "proj", "fc1", "fc2")
    model = ("qkv", "proj", "fc1+gelu", "fc2")
    tot = sum(rows[k]["packed_us"] for k in plain)
    lib = sum(rows[k]["library_us"] for k in plain)
    print(json.dumps({"metric": "ViT-B/16 q2 layer forward, packed kernel vs dense library GEMM on the decoded weight",
                      "m": m, "steps": steps, "block_packed_us": round(tot, 1), "block_library_us": round(lib, 1),
                      "block_with_gelu_packed_us": round(sum(rows[k]["packed_us"] for k in model), 1),
                      "block_with_gelu_library_us": round(sum(rows[k]["library_us"] for k in model), 1),
                      "layers": rows}))
    return 0


def grad_x_bench(m: int, steps: int) -> int:
    """Input gradient of the ViT-B/16 q2 layers at m rows (default bs256 x
    197 tokens) on the packed blob (rpfq_wide_linear_grad_x) against the
    dense library GEMM on the decoded weight (torch.matmul, hipBLASLt):
    fp16 grad_y into fp16 grad_x, and float32 grad_y into float32 grad_x
    (the float32 QAT backward: packed fp16 MFMA operands after the per-row
    scaling vs the float32 library GEMM).  HIP events over `steps` calls on
    the current stream; prints one JSON line."""
    import torch

    def timed(fn):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    rows = {}
    g = torch.Generator(device="cuda").manual_seed(3)
    for name, n_c, k_c in GRAD_SHAPES:
        pw = stream_layer(k_c, n_c, 1)[0]
        pw.adjoint()
        a16 = pw.decode(round_fp16=True)
        flops = 2 * m * 2 * n_c * 2 * k_c
        row = {"n_complex": n_c, "k_complex": k_c}
        for tag, dt in (("fp16", torch.float16), ("f32", torch.float32)):
            gy = torch.randn(m, 2 * n_c, device="cuda", generator=g).to(dt)
            a = a16.to(dt)
            us_packed = timed(lambda: pw.grad_x(gy, dt))
            us_dense = timed(lambda: torch.matmul(gy, a))
            row[tag] = {"packed_us": round(us_packed, 1), "packed_tflops": round(flops / us_packed / 1e6, 1),
                        "frac": round(flops / us_packed / 1e6 / 2500.0, 4), "dense_library_us": round(us_dense, 1)}
            del gy, a
        rows[name] = row
        print(f"# grad_x {name}: {row}", file=sys.stderr, flush=True)
        del pw, a16
        torch.cuda.empty_cache()
    tot = {t: sum(r[t]["packed_us"] for r in rows.values()) for t in ("fp16", "f32")}
    dense = {t: sum(r[t]["dense_library_us"] for r in rows.values()) for t in ("fp16", "f32")}
    flops = sum(2 * m * 2 * n * 2 * k for _, n, k in GRAD_SHAPES)
    print(json.dumps({"metric": "grad_x TFLOP/s, ViT-B/16 q2 layer shapes (one block)", "m": m, "steps": steps,
                      "value": round(flops / tot["fp16"] / 1e6, 1), "unit": "TFLOP/s",
                      "roofline": {"bound": "mfma", "peak": 2500.0, "frac": round(flops / tot["fp16"] / 1e6 / 2500.0, 4),
                                   "kernel": "rpfq::wide_grad_x_kernel"},
                      "block_us": tot, "dense_library_block_us": dense, "layers": rows}))
    return 0


def train_bench(cfg_name: str, batch: int, steps: int, warmup: int, act_quant: bool, modes=("hip", "torch"),
                amp: bool = False):
    """Quantization-aware training steps of the configured model (float32,
    or with amp the forward under fp16 autocast and a gradient scaler as the
    reference trainer's --amp runs it; rotation at the family default, SGD):
    forward with every Linear
    quantized from its float32 master weight, backward with straight-through
    gradients, optimizer step.  'hip' runs the weight quantizer and the act
    quant as HIP kernels (rpfq_quantize_wide, rpfq_act_quant); 'hip_pgrad'
    also takes each layer's input gradient on the packed blob of the step's
    codes (rpfq_wide_linear_grad_x, RPFQ_QAT_PACKED_GRAD=1); 'torch' runs
    the reference formulation in torch ops on the GPU.  Also times the weight
    quantization of all layers alone (no grad).  Prints one JSON line."""
    import torch
    import torch.nn.functional as F
    import quant_models as qm
    from quant_models import quant_i
    from quant_models.inference import quant_layers

    name, _, img, _, seed, desc = CONFIGS[cfg_name]
    out = {}
    for mode in modes:
        quant_i.HIP_QAT = mode in ("hip", "hip_pgrad")
        quant_i.QAT_PACKED_GRAD = "1" if mode == "hip_pgrad" else "0"
        torch.manual_seed(seed)
        model = qm.create_model(name, img_size=img, quant_method_u="complex_phase_v2",
                                quant_method_w="complex_phase_v2", enable_act_quant=act_quant).cuda().train()
        opt = torch.optim.SGD(model.parameters(), lr=1e-4, momentum=0.9)
        g = torch.Generator(device="cuda").manual_seed(seed)
        x = torch.randn(batch, 3, img, img, device="cuda", generator=g)
        labels = torch.randint(0, 1000, (batch,), device="cuda", generator=g)

        scaler = torch.amp.GradScaler("cuda") if amp else None

        def step():
            opt.zero_grad(set_to_none=True)
            if scaler is None:
                loss = F.cross_entropy(model(x), labels)
                loss.backward()
                opt.step()
                return loss
            with torch.autocast("cuda", dtype=torch.float16):
                loss = F.cross_entropy(model(x), labels)
            scaler.scale(loss).backward()
            scaler.step(opt)
            scaler.update()
            return loss

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        layers = [layer for _, layer in quant_layers(model)]
        probe = torch.zeros(1, device="cuda")
        with torch.no_grad():
            for _ in range(2):
                for layer in layers:
                    if mode != "torch":
                        quant_i._HipWideQuantSTE.apply(layer.weight, layer.quantizer_u.rotation_angle,
                                                       layer.quantizer_w.rotation_angle, layer._hip_qat_spec(probe))
                    else:
                        layer.quantized_weight()
            torch.cuda.synchronize()
            tq = time.perf_counter()
            for layer in layers:
                if mode != "torch":
                    quant_i._HipWideQuantSTE.apply(layer.weight, layer.quantizer_u.rotation_angle,
                                                   layer.quantizer_w.rotation_angle, layer._hip_qat_spec(probe))
                else:
                    layer.quantized_weight()
            torch.cuda.synchronize()
            tq = time.perf_counter() - tq
        out[mode] = {"images_per_s": round(batch * steps / dt, 2), "ms_per_step": round(1e3 * dt / steps, 3),
                     "weight_quant_ms": round(1e3 * tq, 3), "layers": len(layers), "final_loss": float(loss)}
        print(f"# train {mode}: {out[mode]}", file=sys.stderr, flush=True)
        del model, opt
        torch.cuda.empty_cache()
    quant_i.HIP_QAT = True
    quant_i.QAT_PACKED_GRAD = os.environ.get("RPFQ_QAT_PACKED_GRAD", "0")
    first = out[modes[0]]
    prec = "fp16 autocast" if amp else "float32"
    print(json.dumps({"metric": f"QAT training images/s {desc}, {prec}, SGD", "value": first["images_per_s"],
                      "unit": "images/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
                      "ms_per_step": first["ms_per_step"], "higher_is_better": True, "data": "synthetic",
                      "config": {"workload": cfg_name, "batch": batch, "act_quant": act_quant, "mode": modes[0],
                                 "amp": amp},
                      "modes": out}))
    return 0


def dominant_kernel(launches):
    """The roofline's kernel: the device kernel (instantiation; a launch
    record's shape[3] names it, +gelu for the GELU-in-store one) with the most
    time among the packed launches.  Returns (its name, (launches, total ms,
    flops, algorithmic bytes) of it, per-kernel summary)."""
    by_kernel = {}
    for e0, e1, fl, by, shape in launches:
        d = by_kernel.setdefault(shape[3] if len(shape) > 3 else "?", [0, 0.0, 0, 0])
        d[0] += 1
        d[1] += e0.elapsed_time(e1)
        d[2] += fl
        d[3] += by
    if not by_kernel:
        return None, (0, 0.0, 0, 0), {}
    dominant = max(by_kernel, key=lambda k: by_kernel[k][1])
    summary = {k: {"launches": v[0], "avg_launch_us": round(1e3 * v[1] / v[0], 2),
                   "tflops": round(v[2] / (v[1] / 1e3) / 1e12, 1) if v[1] > 0 else None}
               for k, v in by_kernel.items()}
    return dominant, tuple(by_kernel[dominant]), summary


RECORD_EVERY = 4  # timed steps per step whose packed launches are bracketed by events


def time_forward(model, x, steps: int, warmup: int, use_graph: bool):
    """Warm up, then time `steps` forwards of model(x) between two events
    (graph replays with use_graph, after checking every replay against the
    eager forward).  The packed launches of every RECORD_EVERY-th timed step
    (steps 0, 4, 8, ...) are bracketed by their own event pairs: each timing
    event is a marker packet on the stream (~2.6 us), so events around every
    launch lengthened the step by ~2% (13.42 vs 13.17 ms, ViT-B/16 bs256,
    same box).  Returns (total ms, per-launch records of the packed layers --
    none under a graph --, the number of recorded steps, the graph or None)."""
    import torch
    from quant_models import ops

    graph = None
    with torch.no_grad():
        for _ in range(warmup):
            model(x)
        torch.cuda.synchronize()
        if use_graph:
            eager = model(x).clone()
            graph = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                with torch.cuda.graph(graph, stream=s):
                    gout = model(x)
            torch.cuda.current_stream().wait_stream(s)
            for _ in range(3):  # every replay, with eager work between, equals the eager forward
                graph.replay()
                torch.cuda.synchronize()
                if not torch.equal(gout, eager):
                    raise AssertionError("graph replay differs from the eager forward")
                model(x)
                torch.cuda.synchronize()

        launches = []
        recorder = lambda e0, e1, fl, by, shape: launches.append((e0, e1, fl, by, shape))  # noqa: E731
        recorded = 0
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for i in range(steps):
            if graph is not None:
                graph.replay()
            else:
                rec = i % RECORD_EVERY == 0
                recorded += rec
                ops.set_launch_recorder(recorder if rec else None)
                model(x)
        end.record()
        torch.cuda.synchronize()
        ops.set_launch_recorder(None)
    return start.elapsed_time(end), launches, recorded, graph


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="vit_b16_q2", choices=sorted(CONFIGS) + ["cplx_fc1"])
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--layer-report", default=None, help="write per-shape kernel timings (JSON) here")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a device copy of this many MiB (counter calibration) and exit")
    ap.add_argument("--read-probe-mib", type=int, default=0,
                    help="only time torch's read (int64 sum) and copy of this many MiB (HBM reference rates) and exit")
    ap.add_argument("--stream-sweep", action="store_true",
                    help="only run the batch-M weight-streaming sweep (M in {1,4,16}, ViT-B/L layer shapes, "
                         ">= --stream-gib GiB of codes per timed pass) and exit")
    ap.add_argument("--stream-gib", type=float, default=1.0)
    ap.add_argument("--stream-modes", default="stacked,rotate")
    ap.add_argument("--stream-ms", default="1,4,16")
    ap.add_argument("--stream-out", default=None, help="write the sweep rows (JSON) here")
    ap.add_argument("--stream-shapes", default=None,
                    help="comma-separated subset of the sweep's layer shapes (e.g. vit_b.fc1)")
    ap.add_argument("--no-stream-line", action="store_true",
                    help="leave the batch-1 streaming summary out of the bench line")
    ap.add_argument("--dtype", default="fp16", choices=["fp16", "bf16"],
                    help="activation dtype of the model forward (and of the batch-1 streaming line)")
    ap.add_argument("--act-quant", action="store_true",
                    help="build the model with 4-bit activation quantization (the reference layer's default)")
    ap.add_argument("--graph", action="store_true",
                    help="capture one forward in a HIP graph and time its replays (launch-bound small batches)")
    ap.add_argument("--layer-probe", default=None, metavar="NC,KC",
                    help="time one q2 layer of N' x K' complex (random codes) on 50,432 fp16 rows instead "
                         "(--steps launches; for counter runs)")
    ap.add_argument("--probe-flags", type=int, default=0,
                    help="rpfq_wide_linear flags of the --layer-probe launches (e.g. 2: no streaming, "
                         "16: the resident-weight kernel)")
    ap.add_argument("--vs-library", action="store_true",
                    help="only time the ViT-B/16 layer forwards on the packed kernel against the dense library GEMM "
                         "on the decoded weight (same box)")
    ap.add_argument("--grad-x", action="store_true",
                    help="time the packed input gradient (rpfq_wide_linear_grad_x) on the ViT-B layer shapes")
    ap.add_argument("--train", action="store_true",
                    help="time quantization-aware training steps (HIP quantizer vs torch ops) instead")
    ap.add_argument("--train-modes", default="hip,hip_pgrad,torch")
    ap.add_argument("--amp", action="store_true", help="with --train: fp16 autocast forward and a gradient scaler")
    ap.add_argument("--no-bf16-line", action="store_true",
                    help="skip the bf16-activation sub-block of the default (fp16) bench line")
    args = ap.parse_args()
    if args.layer_probe:
        return layer_probe(*(int(v) for v in args.layer_probe.split(",")), args.batch or 50432, args.steps,
                           args.probe_flags)
    if args.grad_x:
        return grad_x_bench(args.batch * 197 if args.batch else 50432, args.steps)
    if args.vs_library:
        return vs_library_bench(args.batch * 197 if args.batch else 50432, args.steps)
    if args.train:
        return train_bench(args.config, args.batch or 64, args.steps, args.warmup, args.act_quant,
                           tuple(args.train_modes.split(",")), amp=args.amp)
    if args.stream_sweep:
        shapes = None if not args.stream_shapes else set(args.stream_shapes.split(","))
        if shapes and not shapes <= set(STREAM_SHAPES):
            print(f"unknown --stream-shapes {sorted(shapes - set(STREAM_SHAPES))}; known: {sorted(STREAM_SHAPES)}",
                  file=sys.stderr)
            return 2
        stream_sweep(tuple(int(v) for v in args.stream_ms.split(",")), tuple(args.stream_modes.split(",")),
                     args.stream_gib, max(1, args.steps), args.stream_out, shapes)
        return 0
    if args.read_probe_mib:
        import torch
        n = args.read_probe_mib << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        out = {"read_probe_bytes": n}
        for name, fn, nbytes in (("int64_sum_read", lambda: src.view(torch.int64).sum(), n),
                                 ("copy_read_write", lambda: dst.copy_(src), 2 * n)):
            fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(args.steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            out[name + "_gbs"] = round(nbytes / (e0.elapsed_time(e1) / args.steps / 1e3) / 1e9, 1)
        print(json.dumps(out))
        return 0
    if args.copy_probe_mib:
        import torch
        src = torch.empty(args.copy_probe_mib << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": src.numel(), "copy_probe_bytes_written": dst.numel(),
                          "launches": args.steps}))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU sharding is part of "
              "this build's design, not of what it benchmarks", file=sys.stderr)
        return 2
    if args.config == "cplx_fc1":
        return bench_config1(args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget)

    import torch
    from quant_models import ops

    act_dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    name, batch, img, codebook, seed, desc = CONFIGS[args.config]
    batch = args.batch or batch
    batch1 = None
    if not args.no_stream_line:
        # batch-1 weight streaming (HBM roof) at the ViT-B fc1 shape; runs before
        # and outside the timed region of the model forward
        k_c, n_c = STREAM_SHAPES["vit_b.fc1"]
        batch1 = {"kernel": "streaming kernels at M = 1 (per case: the one rpfq_wide_linear_kernel reports)",
                  "bound": "hbm", "peak": PEAK_HBM_GBS,
                  "unit": "GB/s", "stacked": stream_case(k_c, n_c, 1, "stacked", 1.0, 10, dtype=act_dtype),
                  "rotate": stream_case(k_c, n_c, 1, "rotate", 1.0, 5, dtype=act_dtype)}
    model = build_model(args.config, args.act_quant, act_dtype)
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(batch, 3, img, img, device="cuda", generator=g).to(act_dtype)

    total_ms, launches, n_rec, graph = time_forward(model, x, args.steps, args.warmup, args.graph)
    ms_step = total_ms / args.steps
    value = batch * args.steps / (total_ms / 1e3)
    dominant, (n_dom, kt, kf, kb), by_kernel = dominant_kernel(launches)
    # graph replays launch no recorded events: no per-launch roofline then
    achieved_tflops = kf / (kt / 1e3) / 1e12 if kt > 0 else None
    per_shape = {}
    for e0, e1, fl, by, shape in launches:
        d = per_shape.setdefault(str(shape), [0, 0.0, fl, by])
        d[0] += 1
        d[1] += e0.elapsed_time(e1)
    if args.layer_report:
        with open(args.layer_report, "w") as f:
            json.dump({k: {"launches": v[0], "avg_us": 1e3 * v[1] / v[0], "tflops": v[2] / (v[1] / v[0] / 1e3) / 1e12,
                           "gbs": v[3] / (v[1] / v[0] / 1e3) / 1e9} for k, v in per_shape.items()}, f, indent=1)

    tokens = {"vit": 197, "deit": 198}.get(name.split("_")[1])
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (N(0,1) images; random-init weights quantized by the reference axis rule, "
                "synthetic per-row scales)",
        "config": {"workload": f"{args.config}: {desc} forward, bs{batch}, {img}x{img}"
                               + (", 4-bit activation quantization" if args.act_quant else "")
                               + (" (HIP graph replay)" if graph is not None else ""),
                   "batch": batch, "tokens": tokens, "packed_layers_per_step": len(launches) // max(1, n_rec)},
        "roofline": {
            "bound": "mfma",
            "achieved": None if achieved_tflops is None else round(achieved_tflops, 2),
            "peak": PEAK_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": None if achieved_tflops is None else round(achieved_tflops / PEAK_F16_TFLOPS, 4),
            "traffic": None,
            "kernel": (f"{dominant}: the packed-layer kernel with the most time in the timed region "
                       f"(its launches in every {RECORD_EVERY}th timed step, from the first; "
                       "+gelu: the instantiation with the GELU in the store)")
                      if dominant else "none (graph replays record no launches)",
            "launches": n_dom,
            "recorded_steps": n_rec,
            "avg_launch_us": round(1e3 * kt / max(1, n_dom), 2),
            "algorithmic_gbs": round(kb / (kt / 1e3) / 1e9, 1) if kt > 0 else None,
            "by_kernel": by_kernel,
        },
        "cpu_baseline": None,
    }
    traffic = os.path.join(ROOT, "profiles", f"wide_linear_{args.config}_traffic.json")
    # the committed counter summary covers the default batch of the eager forward
    if os.path.exists(traffic) and batch == CONFIGS[args.config][1] and graph is None:
        with open(traffic) as f:
            line["roofline"]["traffic"] = json.load(f).get("bytes_per_launch")
    if batch1 is not None:
        line["batch1_stream"] = batch1
    if args.dtype == "fp16" and not args.no_bf16_line and not args.graph:
        # the configs' stated bf16 activations: the same forward on a bf16 copy
        # of the model, timed like the headline (after it, outside its region)
        del model
        torch.cuda.empty_cache()
        model_b = build_model(args.config, args.act_quant, torch.bfloat16)
        xb = x.to(torch.bfloat16)
        tb, lb, _, _ = time_forward(model_b, xb, args.steps, args.warmup, False)
        dom_b, (n_b, ktb, kfb, _), by_b = dominant_kernel(lb)
        ach_b = kfb / (ktb / 1e3) / 1e12 if ktb > 0 else None
        line["bf16"] = {"value": round(batch * args.steps / (tb / 1e3), 2), "unit": "images/s",
                        "ms_per_step": round(tb / args.steps, 4), "steps": args.steps, "warmup": args.warmup,
                        "dtype": "bf16",
                        "roofline": {"bound": "mfma", "achieved": None if ach_b is None else round(ach_b, 2),
                                     "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                                     "frac": None if ach_b is None else round(ach_b / PEAK_F16_TFLOPS, 4),
                                     "kernel": dom_b, "launches": n_b,
                                     "avg_launch_us": round(1e3 * ktb / max(1, n_b), 2), "by_kernel": by_b}}
        model = model_b
        x = xb
    if not args.no_cpu_baseline:
        rows = rows_per_image(model, x[:1])
        line["cpu_baseline"] = cpu_baseline(model, rows, args.cpu_budget)
        line["cpu_baseline"]["as_is"] = cpu_baseline_as_is(model, rows, batch, line["cpu_baseline"]["value"],
                                                           4 if args.act_quant else 0, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
