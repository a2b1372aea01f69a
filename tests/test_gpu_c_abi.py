"""The C consumer of include/mxq.h on the GPU (tests/c_abi/mxq_c_test, linked by
build()): it loads x and a quantized triple from a safetensors file into device
memory through the library's loader, runs the quantized matmul on the MLX layout
and on a tiled copy, checks the untiled bits against the file, and writes both
outputs. Here they are compared with the oracle (tight bound against
orc_qmm_f64_bf16w, 2e-2 against exact fp64) and with each other (bit-identical:
both run the same MFMA arithmetic for M > 64, K % 64 == 0)."""
import os
import subprocess

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from tests.gpu_util import assert_tight, spec_metric
from tests.test_gpu_matmul import make_case

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "mxq_c_test")


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("M,N,K,gs,bits", [(300, 320, 1024, 64, 6), (2, 256, 4096, 64, 4),
                                           (130, 192, 512, 32, 3)])
def test_c_program_qmm(dev, O, tmp_path, M, N, K, gs, bits):
    assert os.path.exists(EXE), "tests/c_abi/mxq_c_test is missing: run build()"
    x, wq, s, b, _ = make_case(O, M, N, K, gs, bits, seed=M + N + bits)
    f = tmp_path / "case.safetensors"
    words = torch.from_numpy(wq.view(np.int32)).view(torch.uint32)  # stored as U32
    save_file({"x": _bf16(x), "blk.lin.weight": words, "blk.lin.scales": _bf16(s),
               "blk.lin.biases": _bf16(b)}, str(f))
    r = subprocess.run([EXE, "qmm", str(f), "blk.lin", str(tmp_path)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"bits={bits} group_size={gs}" in r.stdout
    ys = {}
    for name in ("y_mlx", "y_tiled"):
        raw = np.fromfile(tmp_path / f"{name}.bin", dtype=np.uint16).reshape(M, N)
        ys[name] = (raw.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    exact = O.qmm_f64(x, wq, s, b, gs, bits)
    for name, y in ys.items():
        if M <= 8:
            assert_tight(y, exact, f"C {name}")
        else:
            assert_tight(y, O.qmm_f64_bf16w(x, wq, s, b, gs, bits), f"C {name}")
        assert spec_metric(y, exact) <= 2e-2, name
    if M > 64:
        np.testing.assert_array_equal(ys["y_mlx"], ys["y_tiled"])
