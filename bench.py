"""Benchmark: ViT-B/16 q2 forward on one MI355X (images/s), with the roofline
of the packed complex-phase GEMM and the CPU oracle timed beside it.

    python bench.py [--steps K] [--warmup W] [--config vit_b16_q2] [--batch B]

One step = one forward pass of the configured model over one synthetic batch
already resident in HBM.  Prints ONE JSON line (see README of the contract):
value = images/s; roofline = the wide-linear kernel (every packed layer
launch in the timed region, timed with HIP events on its launch stream);
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


def build_model(cfg_name: str):
    import torch
    import quant_models as qm
    from quant_models import _native as N
    from quant_models.inference import load_synthetic_codes, prepare_inference

    name, _, img, codebook, seed, _ = CONFIGS[cfg_name]
    torch.manual_seed(seed)
    model = qm.create_model(name, img_size=img, quant_method_u="complex_phase_v2",
                            quant_method_w="complex_phase_v2", enable_act_quant=False, enable_rotation=False)
    cb = N.CB_PSK16 if codebook == "psk16" else N.CB_AXIS
    load_synthetic_codes(model, seed, cb)
    prepare_inference(model, "cuda", torch.float16)
    return model


def rows_per_image(model, x):
    """Rows each packed layer sees per image in one forward (pre-hooks)."""
    import torch
    from quant_models.inference import quant_layers

    rows, hooks = {}, []
    for name, layer in quant_layers(model):
        def hook(mod, inp, name=name):
            rows[name] = inp[0].numel() // inp[0].shape[-1] // x.shape[0]
        hooks.append(layer.register_forward_pre_hook(hook))
    with torch.no_grad():
        model(x[:1].repeat(x.shape[0], 1, 1, 1) if x.shape[0] > 1 else x)
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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="vit_b16_q2", choices=sorted(CONFIGS))
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--layer-report", default=None, help="write per-shape kernel timings (JSON) here")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a device copy of this many MiB (counter calibration) and exit")
    args = ap.parse_args()
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
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU sharding is a design "
              "note in DESIGN.md, not a benchmark of this build", file=sys.stderr)
        return 2

    import torch
    from quant_models import ops

    name, batch, img, codebook, seed, desc = CONFIGS[args.config]
    batch = args.batch or batch
    model = build_model(args.config)
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(batch, 3, img, img, device="cuda", generator=g).to(torch.float16)

    with torch.no_grad():
        for _ in range(args.warmup):
            model(x)
        torch.cuda.synchronize()

        launches = []
        ops.set_launch_recorder(lambda e0, e1, fl, by, shape: launches.append((e0, e1, fl, by, shape)))
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            out = model(x)
        end.record()
        torch.cuda.synchronize()
        ops.set_launch_recorder(None)

    total_ms = start.elapsed_time(end)
    ms_step = total_ms / args.steps
    value = batch * args.steps / (total_ms / 1e3)
    kt = sum(e0.elapsed_time(e1) for e0, e1, *_ in launches)
    kf = sum(fl for _, _, fl, _, _ in launches)
    kb = sum(by for _, _, _, by, _ in launches)
    achieved_tflops = kf / (kt / 1e3) / 1e12
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
        "dtype": "fp16",
        "data": "synthetic (N(0,1) images; random-init weights quantized by the reference axis rule, "
                "synthetic per-row scales)",
        "config": {"workload": f"{args.config}: {desc} forward, bs{batch}, {img}x{img}",
                   "batch": batch, "tokens": tokens, "packed_layers_per_step": len(launches) // args.steps},
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved_tflops, 2),
            "peak": PEAK_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved_tflops / PEAK_F16_TFLOPS, 4),
            "traffic": None,
            "kernel": "rpfq::wide_linear_dma_kernel (fp16 x, K' % 32 == 0, M >= 128; else "
                      "rpfq::wide_linear_kernel): all packed-layer launches in the timed region",
            "launches": len(launches),
            "avg_launch_us": round(1e3 * kt / max(1, len(launches)), 2),
            "algorithmic_gbs": round(kb / (kt / 1e3) / 1e9, 1),
        },
        "cpu_baseline": None,
    }
    traffic = os.path.join(ROOT, "profiles", f"wide_linear_{args.config}_traffic.json")
    if os.path.exists(traffic):
        with open(traffic) as f:
            line["roofline"]["traffic"] = json.load(f).get("bytes_per_launch")
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(model, rows_per_image(model, x[:1]), args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
