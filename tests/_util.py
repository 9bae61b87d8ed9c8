"""Shared helpers for the tests: bf16 bit patterns <-> numpy / torch, error metrics."""
import numpy as np


def bf16_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def torch_bf16_bits(t):
    """bf16 torch tensor (any device) -> numpy uint16 bit patterns."""
    import torch

    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def to_torch_bf16(bits, device="cuda"):
    import torch

    a = np.ascontiguousarray(bits, np.uint16)
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)


def to_torch_u32(words, device="cuda"):
    import torch

    a = np.ascontiguousarray(words, np.uint32)
    return torch.from_numpy(a.view(np.int32)).to(device)


def u32_of(t):
    return t.detach().contiguous().cpu().numpy().view(np.uint32)


def max_rel_err(y, ref):
    """max |y - ref| / max |ref|  (normwise relative error, the op tolerance metric)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))


def bf16_ulp_diff(a_bits, b_bits):
    """Distance in bf16 ulps between two bf16 bit arrays (sign-magnitude aware)."""
    def key(h):
        h = np.asarray(h, np.uint16).astype(np.int32)
        return np.where(h & 0x8000, -(h & 0x7FFF), h & 0x7FFF)

    return np.abs(key(a_bits) - key(b_bits))


def l2_rel_err(y, ref):
    """||y - ref||_2 / ||ref||_2  (the end-to-end logits tolerance metric)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / (den if den > 0 else 1.0))
