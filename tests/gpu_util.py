"""Host<->device helpers and tolerance checks shared by the GPU tests."""
import numpy as np
import torch


def dev_bf16(u16, dev):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).to(dev).view(torch.bfloat16)


def dev_words(u32, dev):
    return torch.from_numpy(np.ascontiguousarray(u32).view(np.int32)).to(dev).view(torch.uint32)


def dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(dev)


def host_bf16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_words(t):
    return t.contiguous().view(torch.int32).cpu().numpy().view(np.uint32)


def host_f32_of_bf16(t):
    return t.float().cpu().numpy().astype(np.float64)


def assert_tight(y, ref, what=""):
    """GPU bf16 output vs an fp64 reference over the same (rounded) weights:
    error = fp32 accumulation (tiny) + one bf16 output rounding (<= 2^-9 |ref|)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(y - ref)
    bound = 2.0 ** -8 * np.abs(ref) + 1e-4 * scale + 1e-6
    bad = err > bound
    assert not bad.any(), (
        f"{what}: {bad.sum()} of {bad.size} outside tolerance; worst err "
        f"{err.max():.3e} (scale {scale:.3e}) at {np.unravel_index(np.argmax(err - bound), err.shape)}")


def spec_metric(y, ref):
    """max|y - ref| / max|ref|, the north-star correctness metric (<= 2e-2)."""
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(y, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def cosine(y, ref):
    a = np.asarray(y, np.float64).ravel()
    b = np.asarray(ref, np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-300))
