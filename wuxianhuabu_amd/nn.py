"""Module types of the quantized-linear path: QuantizedLinear and MfLinear.

QuantizedLinear mirrors MLXNN's QuantizedLinear as the reference uses it:
    QuantizedLinear(inDims, outDims, bias:, groupSize:, bits:)
        `model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:177-188, 387-388`
    parameters weight (uint32 packed), scales, biases, optional bias, loaded by
    update(parameters:) from keys X.weight / X.scales / X.biases
        `model/4 组装实现&调用/ltx2.5-(ltx专属).swift:576-581`
    callAsFunction(x) = quantizedMatmul(x, weight, scales, biases, transpose: true,
        groupSize, bits) + bias

MfLinear mirrors the reference's own wrapper (`model/minimax h3/H3Common.swift:283-377`):
load() infers bits = 32*wCols/in and groupSize = in/sCols, casts scales/biases
to the compute dtype; forward() casts x to bf16, runs the quantized matmul,
then adds the bias. Here the bias add is fused into the kernel epilogue (added
in fp32 before the single bf16 rounding).

Both hold ONE resident copy of the weight. It starts as the MLX triple; when the
geometry allows (K % 64 == 0, bf16 scales/biases) the first call tiles it
(mxq_tile, the same bits reordered) and the triple is dropped, so a layer costs
K*N*bits/8 bytes of codes plus 4*N*K/gs bytes of scales and biases either way.
Calls then run the tiled kernels, whose results are bit-identical to the
MLX-layout kernels. The parameters keep their MLX meaning: reading weight /
scales / biases (MfLinear: w / scales / biases) returns the triple, rebuilt from
the tiled copy by mxq_untile (a temporary the caller owns); assigning one of
them, or update(), replaces the triple and drops the tiled copy, which the next
call rebuilds. `tiled=False` keeps the triple and runs the MLX-layout kernels.
"""
import math

import torch

from . import ops
from .weights import get_quantized, infer_geometry


class _OneCopy:
    """The resident copy of a quantized weight: `_triple` (MLX layout) or `_tw` (tiled),
    never both once tiled (H3MlpW may hand a holder its fc1 pairs-tiled copy)."""

    _triple = None
    _tw = None

    def _parts(self):
        if self._triple is not None:
            return self._triple
        if self._tw is not None:
            return ops.untile(self._tw)
        return (None, None, None)

    def _set_part(self, i, value):
        parts = list(self._parts())
        parts[i] = value
        self._triple = tuple(parts)
        self._tw = None

    def _adopt(self, tw):
        """Hold `tw` (built from this holder's triple) in place of the triple."""
        self._tw = tw
        self._triple = None

    def _plain_tiled(self, K, group_size, bits, enabled):
        """The plain tiled copy, built from the triple (and replacing it) on first use;
        None when tiling is off or the geometry does not allow it."""
        if self._tw is not None:  # a pairs-tiled copy serves only H3MlpW's fused call
            return None if self._tw.swiglu else self._tw
        if not enabled or self._triple is None:
            return None
        w, s, b = self._parts()
        if not ops.tiled_supported(K, group_size, bits, s.dtype):
            return None
        self._adopt(ops.tile(w, s, b, group_size, bits))
        return self._tw


def _part(i, doc):
    return property(lambda self: self._parts()[i], lambda self, v: self._set_part(i, v),
                    doc=doc)


class QuantizedLinear(_OneCopy):
    tiled = True  # class default; from_weights / __init__ may override per instance

    weight = _part(0, "packed codes, uint32 [out, in*bits/32] (MLX layout)")
    scales = _part(1, "per-group scales [out, in/group_size]")
    biases = _part(2, "per-group biases [out, in/group_size]")

    def __init__(self, input_dims, output_dims, bias=True, group_size=64, bits=4,
                 device="cuda", seed=None, tiled=True):
        # MLXNN initialises uniform(-1/sqrt(in), 1/sqrt(in)) and quantizes it.
        self.tiled = bool(tiled)
        self.input_dims = int(input_dims)
        self.output_dims = int(output_dims)
        self.group_size = int(group_size)
        self.bits = int(bits)
        g = torch.Generator(device="cpu")
        if seed is not None:
            g.manual_seed(seed)
        scale = math.sqrt(1.0 / self.input_dims)
        w = (torch.rand(self.output_dims, self.input_dims, generator=g) * 2 - 1) * scale
        w = w.to(device=device, dtype=torch.bfloat16)
        self._triple = ops.quantized(w, self.group_size, self.bits)
        self.bias = (torch.zeros(self.output_dims, dtype=torch.bfloat16, device=device)
                     if bias else None)

    @classmethod
    def from_weights(cls, weight, scales, biases, bias=None, group_size=64, bits=4,
                     tiled=True):
        """Wrap an existing packed triple (as update(parameters:) does)."""
        obj = cls.__new__(cls)
        obj.tiled = bool(tiled)
        obj._triple = (weight, scales, biases)
        obj._tw = None
        obj.bias = bias
        obj.group_size = int(group_size)
        obj.bits = int(bits)
        obj.output_dims = int(weight.shape[0])
        obj.input_dims = int(weight.shape[1] * 32 // bits)
        return obj

    @classmethod
    def from_linear(cls, weight, bias=None, group_size=64, bits=4, mode="mlx_edge"):
        """Quantize a dense [out, in] weight (MLXNN QuantizedLinear.from(linear:))."""
        wq, s, b = ops.quantized(weight.contiguous(), group_size, bits, mode=mode)
        return cls.from_weights(wq, s, b, bias, group_size, bits)

    def update(self, parameters):
        """Load weight/scales/biases/bias from a mapping of tensors."""
        for key in ("weight", "scales", "biases"):
            if key not in parameters:
                raise KeyError(f"QuantizedLinear.update: missing '{key}'")
        self._triple = (parameters["weight"], parameters["scales"], parameters["biases"])
        self._tw = None
        if "bias" in parameters:
            self.bias = parameters["bias"]
        self.output_dims = int(self._triple[0].shape[0])
        self.input_dims = int(self._triple[0].shape[1] * 32 // self.bits)
        return self

    @property
    def shape(self):
        return (self.output_dims, self.input_dims)

    def tiled_weight(self):
        """The tiled copy of the weight, built on first use (it then replaces the
        triple); None when the geometry does not allow one or tiling is off."""
        return self._plain_tiled(self.input_dims, self.group_size, self.bits, self.tiled)

    def __call__(self, x):
        tw = self.tiled_weight()
        if tw is not None and x.dtype == torch.bfloat16 and x.shape[-1] == tw.K:
            return ops.tiled_matmul(x, tw, bias=self.bias)
        w, s, b = self._parts()  # argument errors come from the MLX-layout operator
        return ops.quantized_matmul(x, w, s, b, transpose=True, group_size=self.group_size,
                                    bits=self.bits, bias=self.bias)

    callAsFunction = __call__


class _Uncached:
    """A weights mapping read without its cache, so that a loaded layer holds the only
    reference to its tensors (SafetensorsFile.get keeps what it reads)."""

    def __init__(self, weights):
        self._w = weights

    def get(self, key):
        return self._w.get_uncached(key)


class MfLinear(_OneCopy):
    """Dense-or-affine-quantized linear, loaded from a weights mapping."""

    scales = _part(1, "per-group scales [out, in/group_size] (quantized layers)")
    biases = _part(2, "per-group biases [out, in/group_size] (quantized layers)")

    def __init__(self, in_dim, out_dim=0):
        self.in_dim = int(in_dim)
        self.out_dim = int(out_dim)
        self.is_quantized = False
        self._dense = None
        self.bias = None
        self.bits = 0
        self.group_size = 0
        self.tiled = True
        self.lora = None  # LoraAdapters (set_lora), the reference's LoraSlot

    @property
    def w(self):
        """packed codes uint32 [out, in*bits/32] (quantized) or the dense weight,
        pre-transposed [in, out]"""
        return self._parts()[0] if self.is_quantized else self._dense

    @w.setter
    def w(self, value):
        if self.is_quantized:
            self._set_part(0, value)
        else:
            self._dense = value

    @classmethod
    def load(cls, weights, prefix, in_features, dtype=torch.bfloat16):
        """`H3Common.swift:312-338`: quantized triple if present, else dense [out, in].
        A mapping with get_uncached (SafetensorsFile) is read without its cache."""
        lin = cls(in_features)
        src = _Uncached(weights) if hasattr(weights, "get_uncached") else weights
        q = get_quantized(src, prefix)
        if q is not None:
            w, s, b = q
            if w.ndim != 2:
                raise ValueError(f"bad file: quantized weight rank {w.ndim}")
            lin.out_dim = int(w.shape[0])
            lin.is_quantized = True
            lin.bits, lin.group_size = infer_geometry(int(w.shape[1]), int(s.shape[1]),
                                                      in_features)
            lin._triple = (w, s.to(dtype).contiguous(), b.to(dtype).contiguous())
        else:
            raw = src.get(prefix + ".weight")
            if raw is None:
                raise KeyError(f"missing weight: {prefix}.weight")
            lin.out_dim = int(raw.shape[0])
            lin._dense = raw.t().to(dtype).contiguous()  # dense, pre-transposed [in, out]
        b = src.get(prefix + ".bias")
        if b is not None:
            lin.bias = b.to(dtype).contiguous()
        return lin

    def set_lora(self, refs):
        """Attach LoRA adapters [(a [in, r], b [r, out], scale), ...]
        (`H3Common.swift:405-434`); an empty list detaches them."""
        refs = list(refs)
        self.lora = ops.LoraAdapters(refs) if refs else None
        return self

    def tiled_weight(self):
        """The plain tiled copy, built on first use (it then replaces the triple)."""
        if not self.is_quantized:
            return None
        return self._plain_tiled(self.in_dim, self.group_size, self.bits, self.tiled)

    def forward(self, x):
        """`H3Common.swift:341-377`: bf16 quantized matmul, + bias, + the LoRA term. On
        tiled weights the LoRA term joins the fp32 accumulators in the kernel, before
        the bias and the one rounding."""
        if self.is_quantized:
            xc = x.to(torch.bfloat16).contiguous()
            tw = self.tiled_weight()
            if tw is not None:
                return ops.tiled_matmul(xc, tw, bias=self.bias, lora=self.lora)
            # the MLX-layout kernels: untiled weights, or fc1 while H3MlpW holds it tiled in
            # gate/up pairs (rebuilt as a temporary triple)
            w, s, b = self._parts()
            if s.dtype != torch.bfloat16:
                raise ValueError("MfLinear: the quantized kernels take bfloat16 scales/biases")
            out = ops.quantized_matmul(xc, w, s, b, transpose=True, group_size=self.group_size,
                                       bits=self.bits, bias=self.bias)
        else:
            # dense branch: not part of the quantized path; plain device matmul
            xc = x.to(self._dense.dtype)
            out = xc @ self._dense
            if self.bias is not None:
                out = out + self.bias
        if self.lora is not None:
            xa = self.lora.xa(xc.reshape(-1, self.in_dim).to(torch.bfloat16))
            out = out + (xa.float() @ self.lora.bt.float().t()).to(out.dtype).reshape(out.shape)
        return out

    __call__ = forward


class LTXFFN:
    """The LTX feed-forward (`model/3模块/ltx2.5专属/ltx主干-(ltx专属).swift:372-401`):
    proj_in -> geluApprox -> proj_out, two QuantizedLinear. With tiled weights the GELU runs
    in proj_in's epilogue (fp32, before the one bf16 rounding), so the [M, ffnDim]
    pre-activation never goes to memory. The IC-LoRA side paths of the reference are not
    part of this path."""

    def __init__(self, dim, ffn_dim, bias=True, group_size=64, bits=4, device="cuda",
                 seed=None, tiled=True):
        self.dim, self.ffn_dim = int(dim), int(ffn_dim)
        self.proj_in = QuantizedLinear(dim, ffn_dim, bias, group_size, bits, device,
                                       None if seed is None else seed, tiled)
        self.proj_out = QuantizedLinear(ffn_dim, dim, bias, group_size, bits, device,
                                        None if seed is None else seed + 1, tiled)

    def __call__(self, x):
        tw = self.proj_in.tiled_weight()
        if tw is not None and x.dtype == torch.bfloat16 and x.shape[-1] == tw.K:
            mid = ops.tiled_matmul(x, tw, bias=self.proj_in.bias, activation="gelu_tanh")
        else:
            mid = torch.nn.functional.gelu(self.proj_in(x).float(),
                                           approximate="tanh").to(torch.bfloat16)
        return self.proj_out(mid)

    callAsFunction = __call__


class H3MlpW:
    """The H3 MLP (`model/minimax h3/H3Transformer.swift:601-629`): fc1 [S, hidden] ->
    [S, 2*ffn] (gate and up fused), silu(gate) * up, fc2. When fc1 is quantized and
    tileable its weight is tiled once in gate/up pairs (mxq_tile_swiglu) and
    silu(gate) * up runs in fc1's epilogue, so the [S, 2*ffn] output never goes to
    memory. fc1's LoRA adapters (MfLinear.set_lora, the reference's fc1Lora) join the
    accumulators before it."""

    def __init__(self, fc1, fc2):
        self.fc1, self.fc2 = fc1, fc2

    @classmethod
    def load(cls, weights, prefix, hidden_size, ffn_hidden, dtype=torch.bfloat16):
        """`H3Transformer.swift:612-616`: fc1 / fc2 MfLinear under prefix.fc1 / prefix.fc2."""
        return cls(MfLinear.load(weights, prefix + ".fc1", hidden_size, dtype),
                   MfLinear.load(weights, prefix + ".fc2", ffn_hidden, dtype))

    def _pairs(self):
        """fc1 tiled in gate/up pairs; fc1 then holds this copy in place of its own."""
        f = self.fc1
        if f._tw is not None and f._tw.swiglu:
            return f._tw
        if not (f.is_quantized and f.tiled and f.out_dim % 2 == 0):
            return None
        w, s, b = f._parts()
        if not ops.tiled_supported(f.in_dim, f.group_size, f.bits, s.dtype):
            return None
        f._adopt(ops.tile(w, s, b, f.group_size, f.bits, swiglu=True))
        return f._tw

    def forward(self, x):
        tw = self._pairs()
        if tw is not None:
            gated = ops.tiled_matmul(x.to(torch.bfloat16).contiguous(), tw, bias=self.fc1.bias,
                                     activation="swiglu", lora=self.fc1.lora)
        else:
            y = self.fc1.forward(x)
            half = y.shape[-1] // 2
            gated = (torch.nn.functional.silu(y[..., :half].float()) *
                     y[..., half:].float()).to(y.dtype)
        return self.fc2.forward(gated)

    __call__ = forward
