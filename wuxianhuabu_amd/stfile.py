"""safetensors files of quantized weights, read through libmxq (mxq_st_*).

SafetensorsFile mirrors the reference's lazy reader H3Weights
(`model/minimax h3/H3Common.swift:181-260`): the header is parsed once (by the
library, from a read-only mapping of the file, as MappedSafetensors does,
`model/3模块/Safetensors-mmap映射-通用.swift:40-135`) and each tensor is read on
demand, straight into device memory through the library's pinned staging
buffers. get() caches like H3Weights.get, get_uncached() does not. A
SafetensorsFile is a weights mapping for MfLinear.load, H3MlpW.load and
weights.get_quantized (both key spellings of the scales/biases).

infer_quant_params() follows the reference's header-only inference
(`model/3模块/模型加载-通用.swift:167-234`): (bits, group_size) candidates from the
packed and scales widths of a few quantized layers, then a score on sampled
rows to pick among widths that fit several pairs (512 packed words and 64
scales fit 2-bit/128, 4-bit/64 and 8-bit/32). The score differs from the
reference's, which reads the codes MSB-first (:256-266, wrong for the MLX
layout), tries 2, 4 and 8 bits only (:214), and ranks by std/max|bias|, which
a narrower misreading can undercut. Here codes are read LSB-first and each
candidate is scored by how its groups use the code range: an affine quantizer
maps each group's extreme weights onto an end code (0 or 2^bits - 1), and the
weights are exchangeable, so code statistics do not depend on the position;
reading 4-bit codes as 8-bit rarely lands on an end, reading them as 2-bit
puts near-uniform low pieces and bell-shaped high pieces at alternating
positions (see _range_use).
"""
import ctypes
import os

import numpy as np
import torch

from . import _lib
from .weights import SUPPORTED_BITS, SUPPORTED_GS, get_quantized, header_candidates

_TORCH = {"BOOL": torch.bool, "U8": torch.uint8, "I8": torch.int8, "I16": torch.int16,
          "U16": torch.uint16, "F16": torch.float16, "BF16": torch.bfloat16,
          "I32": torch.int32, "U32": torch.uint32, "F32": torch.float32, "I64": torch.int64,
          "U64": torch.uint64, "F64": torch.float64}


class SafetensorsFile:
    def __init__(self, path, device="cuda"):
        self.path = os.fspath(path)
        self.device = torch.device(device)
        h = ctypes.c_void_p()
        L = _lib.lib()
        _lib.check(L.mxq_st_open(self.path.encode(), ctypes.byref(h)))
        self._h = h
        n = L.mxq_st_count(h)
        self._keys = [L.mxq_st_key(h, i).decode() for i in range(n)]
        self._cache = {}

    # ---- mapping protocol
    def keys(self):
        return list(self._keys)

    def __contains__(self, key):
        return key in self._keys

    def __len__(self):
        return len(self._keys)

    def info(self, key):
        """(dtype name, shape, nbytes) of `key`."""
        L = _lib.lib()
        dt = ctypes.create_string_buffer(16)
        nd = ctypes.c_int()
        shape = (ctypes.c_int64 * 8)()
        nb = ctypes.c_int64()
        _lib.check(L.mxq_st_info(self._handle(), key.encode(), dt, ctypes.byref(nd), shape,
                                 ctypes.byref(nb)))
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value)), nb.value

    def get(self, key, device=None):
        """The tensor `key` on `device` (default: the file's), cached; None if absent."""
        if key not in self._keys:
            return None
        dev = torch.device(device) if device is not None else self.device
        ck = (key, str(dev))
        if ck not in self._cache:
            self._cache[ck] = self.get_uncached(key, dev)
        return self._cache[ck]

    def get_uncached(self, key, device=None):
        if key not in self._keys:
            return None
        dev = torch.device(device) if device is not None else self.device
        dt, shape, nbytes = self.info(key)
        if dt not in _TORCH:
            raise ValueError(f"[safetensors] tensor '{key}' has unsupported dtype {dt}.")
        out = torch.empty(shape, dtype=_TORCH[dt], device=dev)
        L = _lib.lib()
        if dev.type == "cuda":
            with torch.cuda.device(dev):
                stream = torch.cuda.current_stream(dev).cuda_stream
                _lib.check(L.mxq_st_read(self._handle(), key.encode(),
                                         ctypes.c_void_p(out.data_ptr()),
                                         ctypes.c_void_p(stream)))
        else:
            _lib.check(L.mxq_st_read_host(self._handle(), key.encode(),
                                          ctypes.c_void_p(out.data_ptr())))
        return out

    def read_bytes(self, key):
        """The tensor's bytes as a host uint8 array, whatever its dtype."""
        _, _, nbytes = self.info(key)
        out = np.empty(nbytes, dtype=np.uint8)
        if nbytes:
            _lib.check(_lib.lib().mxq_st_read_host(self._handle(), key.encode(),
                                                   out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def get_quantized(self, prefix):
        """(weight, scales, biases) for `prefix` in either key spelling, or None."""
        return get_quantized(self, prefix)

    def clear_cache(self):
        self._cache.clear()

    # ---- header-only quantization parameters
    def infer_quant_params(self, samples=3, scored=2):
        """(bits, group_size) shared by the file's quantized layers, or None when it has
        none; ValueError if the widths admit no supported pair."""
        layers = []
        for k in self._keys:
            if not k.endswith(".weight"):
                continue
            dt, shape, _ = self.info(k)
            if dt != "U32" or len(shape) != 2 or shape[0] == 0:  # no rows: nothing to score
                continue
            base = k[: -len("weight")]
            for sk, bk in ((base + "scales", base + "biases"),
                           (k + ".scales", k + ".biases")):
                if sk in self._keys and bk in self._keys and len(self.info(sk)[1]) == 2:
                    layers.append((k, sk, bk, shape[1], self.info(sk)[1][1]))
                    break
            if len(layers) >= samples:
                break
        if not layers:
            return None
        cands = [c for c in header_candidates(layers[0][3], layers[0][4])
                 if all(c in header_candidates(w2, s2) for _, _, _, w2, s2 in layers)]
        if not cands:
            raise ValueError(f"[safetensors] packed width {layers[0][3]} and scales width "
                             f"{layers[0][4]} fit no supported (bits, group_size).")
        if len(cands) == 1:
            return cands[0]
        best, best_score = None, float("inf")
        for bits, gs in cands:
            score = float(np.mean([_range_use(self, wk, sk, bits, gs) for wk, sk, _, _, _ in
                                   layers[:scored]]))
            if score < best_score:
                best, best_score = (bits, gs), score
        return best

    # ---- lifetime
    def _handle(self):
        if self._h is None:
            raise ValueError("[safetensors] the file is closed.")
        return self._h

    def close(self):
        if getattr(self, "_h", None) is not None:
            _lib.lib().mxq_st_close(self._h)
            self._h = None
        self._cache = {}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _codes(w, bits):
    """LSB-first bitstream: code k of each row is bits [k*bits, k*bits + bits)."""
    K = w.shape[1] * 32 // bits
    bitpos = np.arange(K, dtype=np.int64) * bits
    word, off = bitpos // 32, (bitpos % 32).astype(np.uint64)
    lo = w[:, word].astype(np.uint64) >> off
    nxt = np.minimum(word + 1, w.shape[1] - 1)
    hi = np.where(off + np.uint64(bits) > 32,
                  w[:, nxt].astype(np.uint64) << (np.uint64(32) - off), np.uint64(0))
    return ((lo | hi) & np.uint64((1 << bits) - 1)).astype(np.int64)


def _range_use(f, wk, sk, bits, gs, rows=16):
    """How far a reading is from what an affine quantizer writes, for one layer:
    - the share of groups without an end code (0 or 2^bits - 1): the quantizer maps each
      group's extreme weight(s) there; reading the codes as wider ones (two b-bit codes
      as one 2b-bit code) rarely lands on an end;
    - the total-variation distance between the code histograms at even and odd (and at
      the four residues mod 4) code positions: the weights are exchangeable, so under the
      right reading these agree; reading 2b-bit codes as b-bit pieces puts the near-
      uniform low pieces and the bell-shaped high pieces at alternating positions."""
    w = f.get_uncached(wk, "cpu")[:rows].contiguous().view(torch.int32).numpy().view(np.uint32)
    q = _codes(w, bits)
    if q.shape[1] % gs:
        return float("inf")
    n = (1 << bits) - 1
    g = q.reshape(q.shape[0], -1, gs)
    miss = 1.0 - float(((g == 0) | (g == n)).any(axis=2).mean())
    tv = 0.0
    for r in (2, 4):
        hs = [np.bincount(q[:, j::r].ravel(), minlength=n + 1) / q[:, j::r].size
              for j in range(r)]
        tv = max(tv, max(0.5 * np.abs(h - hs[0]).sum() for h in hs[1:]))
    return miss + tv


__all__ = ["SafetensorsFile", "SUPPORTED_BITS", "SUPPORTED_GS"]
