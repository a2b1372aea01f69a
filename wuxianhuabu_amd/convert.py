"""Producers of the quantized triple.

quantize_checkpoint(src, dst, group_size=64, bits=4)
    The reference's offline repacker (`model/minimax h3/tools/quantize_h3_g64.py:92-156`):
    every tensor that passes should_quant (BF16, 2-D, last dimension >= group_size and
    a multiple of it; :92-99) becomes the triple `k` (U32 packed codes), `k.scales` and
    `k.biases` (BF16), as mx.quantize writes it (:132-136); every other tensor is copied
    byte for byte. The quantization runs on the GPU (mxq_quantize, mlx's algorithm by
    default). Like the reference it streams tensor by tensor, and it also writes that
    way: the output header is computed from the shapes alone, then each tensor is read
    into HBM through libmxq's loader, quantized, and appended, so neither file is ever
    held whole in host or device memory (the reference collects every output array
    before mx.save_safetensors, :156).
quantize_module(module, filter=None, group_size=64, bits=4)
    MLXNN's quantize(model:filter:) as the reference calls it
    (`Packages/z-image-swift/Sources/ZImage/Weights.swift:30-37`), over a torch module
    tree: each torch.nn.Linear for which filter(path, module) returns parameters is
    replaced by a QuantizedLinearModule.

Command line, with the reference's flags:
    python -m wuxianhuabu_amd.convert --src A.safetensors --dst B.safetensors
        [--bits 4] [--group-size 64] [--mode mlx_edge|minmax] [--dry-run]
"""
import argparse
import json
import os
import time

import numpy as np
import torch

from . import ops
from .nn import QuantizedLinear
from .stfile import SafetensorsFile


def should_quant(dtype, shape, group_size=64):
    """The repacker's rule (`quantize_h3_g64.py:92-99`): BF16, 2-D, last dimension at
    least the group size and a multiple of it. Everything else is kept: 1-D norms and
    biases, pruned [96768, 8] adaLN factor tables, F32 lookup tables."""
    return (dtype == "BF16" and len(shape) == 2 and shape[-1] >= group_size and
            shape[-1] % group_size == 0)


def _plan(f, group_size, bits):
    """[(source key, quantize?, [(out key, dtype, shape, nbytes), ...])] in source order."""
    plan = []
    for k in f.keys():
        dt, shape, nbytes = f.info(k)
        if should_quant(dt, shape, group_size):
            n, kdim = shape
            sb = (n, kdim // group_size)
            outs = [(k, "U32", (n, kdim * bits // 32), n * kdim * bits // 8),
                    (k + ".scales", "BF16", sb, sb[0] * sb[1] * 2),
                    (k + ".biases", "BF16", sb, sb[0] * sb[1] * 2)]
            plan.append((k, True, outs))
        else:
            plan.append((k, False, [(k, dt, tuple(shape), nbytes)]))
    return plan


def _header(plan):
    entries, off = {"__metadata__": {"format": "mlx"}}, 0
    for _, _, outs in plan:
        for key, dt, shape, nbytes in outs:
            entries[key] = {"dtype": dt, "shape": list(shape),
                            "data_offsets": [off, off + nbytes]}
            off += nbytes
    raw = json.dumps(entries, separators=(",", ":")).encode("utf-8")
    raw += b" " * (-len(raw) % 8)  # the data area starts 8-byte aligned
    return raw, off


def _host_bytes(t):
    if not t.numel():
        return b""
    if t.dtype == torch.uint32:
        t = t.view(torch.int32)
    return t.contiguous().cpu().view(torch.uint8).numpy().tobytes()


def quantize_checkpoint(src, dst, group_size=64, bits=4, mode="mlx_edge", dry_run=False,
                        device="cuda", log=None):
    """Quantize every should_quant tensor of `src` into MLX triples and write `dst`.
    Returns {"quantized": nq, "kept": nk, "entries": nq*3 + nk, "bytes": size of dst}
    ("bytes" is what would be written when dry_run)."""
    log = log or (lambda msg: None)
    t0 = time.time()
    with SafetensorsFile(src, device=device) as f:
        plan = _plan(f, group_size, bits)
        nq = sum(1 for _, q, _ in plan if q)
        stats = {"quantized": nq, "kept": len(plan) - nq, "entries": 3 * nq + len(plan) - nq}
        header, data_bytes = _header(plan)
        stats["bytes"] = 8 + len(header) + data_bytes
        log(f"{len(plan)} source tensors: quantize {nq} ({3 * nq} entries), keep "
            f"{len(plan) - nq}, {stats['entries']} entries")
        if dry_run:
            return stats
        os.makedirs(os.path.dirname(os.path.abspath(dst)), exist_ok=True)
        with open(dst, "wb") as out:
            out.write(np.uint64(len(header)).tobytes())
            out.write(header)
            for i, (k, quant, outs) in enumerate(plan):
                if quant:
                    w = f.get_uncached(k, device)
                    wq, s, b = ops.quantized(w, group_size, bits, mode=mode)
                    del w
                    parts = (wq, s, b)
                else:
                    parts = (torch.from_numpy(f.read_bytes(k)),)
                for (_, _, _, nbytes), t in zip(outs, parts):
                    data = _host_bytes(t)
                    if len(data) != nbytes:
                        raise RuntimeError(f"[convert] '{k}': {len(data)} bytes, planned "
                                           f"{nbytes}")
                    out.write(data)
                if (i + 1) % 25 == 0 or i + 1 == len(plan):
                    log(f"  {i + 1}/{len(plan)} ({time.time() - t0:.0f}s)")
    stats["bytes"] = os.path.getsize(dst)
    return stats


class QuantizedLinearModule(torch.nn.Module):
    """A QuantizedLinear where a torch module tree expects a child module."""

    def __init__(self, q):
        super().__init__()
        self.q = q

    def forward(self, x):
        return self.q(x)

    def extra_repr(self):
        q = self.q
        return (f"input_dims={q.input_dims}, output_dims={q.output_dims}, "
                f"group_size={q.group_size}, bits={q.bits}, bias={q.bias is not None}")


def _params(res, group_size, bits, mode):
    """A filter's answer -> (group_size, bits, mode), or None to keep the layer."""
    if res is None or res is False:
        return None
    if res is True:
        return group_size, bits, mode
    gs, b, md = (tuple(res) + (group_size, bits, mode)[len(tuple(res)):])[:3]
    return gs, b, "mlx_edge" if md == "affine" else md  # MLX's .affine mode


def quantize_module(module, filter=None, group_size=64, bits=4, mode="mlx_edge", prefix=""):
    """Replace, in place, each torch.nn.Linear under `module` whose filter(path, module)
    returns True or (group_size, bits[, mode]) by a QuantizedLinearModule (None / False
    keeps it; no filter quantizes every Linear whose input width the group size
    divides, as quantize(model:) does). Paths are dotted child names, as MLX's.
    Returns the list of quantized paths."""
    done = []
    for name, child in list(module.named_children()):
        path = f"{prefix}.{name}" if prefix else name
        if isinstance(child, torch.nn.Linear):
            if filter is None:
                p = (group_size, bits, mode) if child.in_features % group_size == 0 else None
            else:
                p = _params(filter(path, child), group_size, bits, mode)
            if p is None:
                continue
            gs, b, md = p
            bias = None if child.bias is None else child.bias.detach().to(torch.bfloat16)
            q = QuantizedLinear.from_linear(child.weight.detach().to(torch.bfloat16),
                                            bias=bias, group_size=gs, bits=b, mode=md)
            setattr(module, name, QuantizedLinearModule(q))
            done.append(path)
        else:
            done += quantize_module(child, filter, group_size, bits, mode, path)
    return done


def main(argv=None):
    ap = argparse.ArgumentParser(description="dense BF16 safetensors -> MLX affine triples")
    ap.add_argument("--src", required=True, help="input safetensors (BF16 weights)")
    ap.add_argument("--dst", required=True, help="output safetensors")
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--group-size", type=int, default=64)
    ap.add_argument("--mode", default="mlx_edge", choices=["mlx_edge", "minmax"])
    ap.add_argument("--dry-run", action="store_true", help="count only, write nothing")
    args = ap.parse_args(argv)
    stamp = lambda msg: print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)  # noqa: E731
    stats = quantize_checkpoint(args.src, args.dst, args.group_size, args.bits, args.mode,
                                args.dry_run, log=stamp)
    stamp(f"done: {stats}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
