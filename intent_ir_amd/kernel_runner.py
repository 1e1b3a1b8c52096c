"""Launch one workload's kernel a fixed number of times (for profilers).

    python -m intent_ir_amd.kernel_runner --config softmax --launches 20 [--copy-mib 512]
    python -m intent_ir_amd.kernel_runner --config matmul --bindings M=4096,N=50257,K=4096 --transpose-b

Inputs are generated on the GPU; launches rotate over enough buffer sets that
reads come from HBM rather than the Infinity Cache (as in bench.py).  With
``--copy-mib`` the run ends with plain device-to-device copies of that size
(torch ``copy_``), whose FETCH_SIZE/WRITE_SIZE readings calibrate the HBM byte
counters against a known transfer.  ``--bindings`` replaces the workload's shape
bindings; ``--transpose-b`` (matmul) gives B as [N, K] with matmul{transpose_b}.
"""

from __future__ import annotations

import argparse
import math
import sys

ROTATE_MIN_BYTES = 640 << 20


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", required=True, choices=["any", "softmax", "layernorm", "gelu", "matmul"])
    ap.add_argument("--launches", type=int, default=20)
    ap.add_argument("--copy-mib", type=int, default=0)
    ap.add_argument("--bindings", default="", help="comma-separated SYMBOL=VALUE overrides, e.g. M=1000,N=4096")
    ap.add_argument("--transpose-b", action="store_true", help="matmul: B given as [N, K] (matmul{transpose_b})")
    args = ap.parse_args(argv)
    if args.transpose_b and args.config != "matmul":
        ap.error("--transpose-b applies to --config matmul only")

    import torch

    from . import lower_intent_to_hip_kernel
    from .configs import WORKLOADS, algorithmic_bytes, gen_device
    from .runtime import launch_lowered, tensor_shapes, torch_dtype

    w = WORKLOADS[args.config]
    b = dict(w.bindings)
    for item in filter(None, args.bindings.split(",")):
        name, _, value = item.partition("=")
        if name not in b:
            ap.error(f"--bindings: {name!r} is not a symbol of {args.config} ({sorted(b)})")
        b[name] = int(value)
    ir = w.ir()
    if args.transpose_b:
        ir["tensors"]["B"]["shape"] = ["N", "K"]
        ir["ops"][0]["attrs"] = {"transpose_b": True}
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    shapes = tensor_shapes(k.io_spec, k.bindings)
    per = algorithmic_bytes(args.config, b)
    nsets = 1 if args.config in ("matmul", "gelu") else max(2, math.ceil(ROTATE_MIN_BYTES / per))
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    sets = []
    for _ in range(nsets):
        bufs = gen_device(args.config, b, torch, g)
        if args.transpose_b:  # same values, read as [N, K]
            bufs["B"] = bufs["B"].reshape(b["N"], b["K"])
        for n in k.output_names:
            bufs[n] = torch.empty(shapes[n], dtype=torch_dtype(k.io_spec["tensors"][n]["dtype"]), device="cuda")
        sets.append(bufs)
    torch.cuda.synchronize()
    for i in range(args.launches):
        launch_lowered(k, sets[i % nsets])
    torch.cuda.synchronize()
    print(f"[runner] {args.config}: {args.launches} launches of {k.kernel_id}, {nsets} buffer sets, "
          f"{per} algorithmic bytes per launch", flush=True)
    if args.copy_mib:
        n = (args.copy_mib << 20) // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[runner] calibration: 3 copies of {args.copy_mib} MiB", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
