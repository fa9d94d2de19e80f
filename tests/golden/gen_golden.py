"""Write golden vectors by running the reference's own Python in this container.

Run once, where /root/reference exists:  python tests/golden/gen_golden.py
It imports two torch-only reference modules by path (never on the GPU box):
  RPFQ-ViT-main/quant_models/quant_i.py            (training-path layer)
  RPFQ-ViTApple/scripts/export_rpfq_vit_to_mlx.py  (packed-format producer)
and records, for seeded inputs, the values closed forms cannot pin
bit-exactly: residual stage values and scales (float32 sums in torch's order),
the fp16-gamma export planes, activation fake-quant at rounding ties, and
full QATLinearComplexPhase.forward outputs.  Only data is written.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

REF = os.environ.get("RPFQ_REFERENCE", "/root/reference")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_v1.npz")

sys.path.insert(0, os.path.join(REF, "RPFQ-ViT-main", "quant_models"))
sys.path.insert(0, os.path.join(REF, "RPFQ-ViTApple", "scripts"))
import quant_i  # noqa: E402
import export_rpfq_vit_to_mlx as export  # noqa: E402


def stage_trace(w_re, w_im, steps):
    """Per-stage (q_re, q_im) of quant_i._residual_quantize, re-driven with the
    reference's own stage function so intermediate values are visible."""
    out = []
    r_re, r_im = w_re, w_im
    for _ in range(steps):
        s_re, s_im = quant_i._quantize_phase_axis(r_re, r_im)
        out.append((s_re.clone(), s_im.clone()))
        r_re = r_re - s_re
        r_im = r_im - s_im
    return out


def main() -> None:
    torch.manual_seed(0)
    g = {}

    # 1) tie-rule table of _axis_masks (every quadrant tie, zero, signed zero)
    vals = torch.tensor([0.0, -0.0, 0.5, -0.5, 1.0, -1.0, 0.25], dtype=torch.float32)
    tr, ti = torch.meshgrid(vals, vals, indexing="ij")
    masks = quant_i._axis_masks(tr.reshape(-1), ti.reshape(-1))
    g["masks_re"] = tr.reshape(-1).numpy()
    g["masks_im"] = ti.reshape(-1).numpy()
    g["masks_out"] = torch.stack(masks).numpy().astype(np.uint8)

    # 2) residual stages (v2 and v4) on a seeded weight, both U and W planes
    weight = torch.randn(64, 96) * 0.02
    weight[0, :8] = 0.0  # exact-zero entries exercise the zero-tie rule
    weight[1, 0], weight[33, 0] = 0.01, 0.01  # a11 == a21 -> w_im = a21 ... ties
    g["w_weight"] = weight.numpy()
    half_o, half_i = 32, 48
    a11, a12 = weight[:half_o, :half_i], weight[:half_o, half_i:]
    a21, a22 = weight[half_o:, :half_i], weight[half_o:, half_i:]
    planes = {
        "u": (0.5 * (a11 + a22), 0.5 * (a21 - a12)),
        "w": (0.5 * (a11 - a22), 0.5 * (a12 + a21)),
    }
    for name, (pr, pi) in planes.items():
        for steps in (2, 4):
            tr_ = stage_trace(pr, pi, steps)
            for s, (qr, qi) in enumerate(tr_):
                g[f"stage_{name}_v{steps}_{s}_re"] = qr.numpy()
                g[f"stage_{name}_v{steps}_{s}_im"] = qi.numpy()
            fr, fi = quant_i._residual_quantize(pr, pi, steps, quant_i._quantize_phase_axis)
            g[f"resq_{name}_v{steps}_re"] = fr.numpy()
            g[f"resq_{name}_v{steps}_im"] = fi.numpy()

    # 3) exporter planes (fp16 gamma feedback, padded to 256) and export A_q
    target = {}
    export.save_quantized_linear(target, "L", weight, torch.zeros(64), 256, 256, 2)
    for k, v in target.items():
        g["exp_" + k.replace(".", "_")] = v.numpy()
    g["exp_aq"] = export.quantized_forward_weight(weight, 2).numpy()
    # unpadded export of a block-aligned shape (K' = 256): gamma [N', 1]
    weight_b = torch.randn(48, 512) * 0.05
    g["expb_weight"] = weight_b.numpy()
    target = {}
    export.save_quantized_linear(target, "L", weight_b, torch.randn(48), 256, 24, 2)
    for k, v in target.items():
        g["expb_" + k.replace(".", "_")] = v.numpy()

    # 4) activation fake-quant with exact rounding ties (x*scale = n + 0.5)
    xr = torch.tensor([[7.0, 0.5, 1.5, 2.5, -0.5, -2.5, 3.5, -7.0],
                       [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
                       [1e-7, -3e-6, 2e-6, 0.0, 1e-6, -1e-6, 5e-7, 4e-6]], dtype=torch.float32)
    xi = torch.randn(3, 8)
    for bits in (2, 4, 8):
        qr, qi = quant_i.ActivationQuantSTE.apply(xr, xi, bits)
        g[f"act{bits}_re"] = qr.numpy()
        g[f"act{bits}_im"] = qi.numpy()
    g["act_xr"] = xr.numpy()
    g["act_xi"] = xi.numpy()
    xa = torch.randn(16, 48) * 3
    g["actr_x"] = xa.numpy()
    qa, qb = quant_i.ActivationQuantSTE.apply(xa[:, :24], xa[:, 24:], 4)
    g["actr_q"] = torch.cat([qa, qb], -1).numpy()

    # 5) full layer forwards on seeded (x, weight, bias)
    x = torch.randn(5, 96)
    bias = torch.randn(64) * 0.1
    g["fwd_x"] = x.numpy()
    g["fwd_bias"] = bias.numpy()
    methods = ["complex_phase_v1", "complex_phase_v2", "complex_phase_v3",
               "complex_phase_v4", "complex_phase_new_v2", "complex_phase_next_v1"]
    for m in methods:
        for act in (False, True):
            for rot in (False, True):
                if m == "complex_phase_next_v1" and rot:
                    continue
                layer = quant_i.QATLinearComplexPhase(
                    quant_method_u=m, quant_method_w=m, enable_act_quant=act,
                    act_num_bits=4, enable_rotation=rot, quant_group_size=32,
                    in_features=96, out_features=64, bias=True)
                with torch.no_grad():
                    layer.weight.copy_(weight)
                    layer.bias.copy_(bias)
                    if rot:
                        layer.quantizer_u.rotation_angle.fill_(0.3)
                        layer.quantizer_w.rotation_angle.fill_(-0.2)
                    y = layer(x)
                    # fused A_q: forward of the identity through a bias-free copy
                    nb = quant_i.QATLinearComplexPhase(
                        quant_method_u=m, quant_method_w=m, enable_act_quant=False,
                        enable_rotation=rot, in_features=96, out_features=64, bias=False)
                    nb.load_state_dict({k: v for k, v in layer.state_dict().items() if k != "bias"})
                    aq = nb(torch.eye(96)).T.contiguous()
                tag = f"{m}_a{int(act)}_r{int(rot)}"
                g[f"fwd_y_{tag}"] = y.numpy()
                g[f"fwd_aq_{tag}"] = aq.numpy()

    np.savez_compressed(OUT, **g)
    print(f"wrote {len(g)} arrays to {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
