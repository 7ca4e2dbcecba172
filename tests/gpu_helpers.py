"""Device-buffer helpers for the GPU parity tests (torch is plumbing only)."""
import numpy as np
import torch

DEV = "cuda:0"

NP_OF = {"f32": np.float32, "bf16": np.uint16, "f16": np.float16}
TORCH_OF = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
TOL = {"f32": 2e-3, "bf16": 2e-2, "f16": 2e-2}  # max-abs bars stated for this path


def to_dev(a: np.ndarray, dtype: str = None) -> torch.Tensor:
    """Uploads a numpy array; uint16 arrays with dtype 'bf16' become bfloat16."""
    a = np.ascontiguousarray(a)
    if dtype == "bf16":
        assert a.dtype == np.uint16
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(a).to(DEV)


def to_host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    return t.contiguous().cpu().numpy()


def as_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    import oracle as O
    if dtype == "bf16":
        return O.bf16_bits_to_f32(a)
    return a.astype(np.float32)


def from_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    """Rounds f32 values to dtype storage (uint16 bits for bf16)."""
    import oracle as O
    if dtype == "bf16":
        return O.f32_to_bf16_bits(a)
    return np.asarray(a, dtype=NP_OF[dtype])


def random_values(rng, shape, dtype: str) -> np.ndarray:
    return from_f32(rng.standard_normal(shape).astype(np.float32), dtype)


def err_report(got: np.ndarray, want: np.ndarray):
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    diff = np.abs(got - want)
    rel = diff.max() / max(np.abs(want).max(), 1e-30)
    return float(diff.max()), float(rel)


def build_tables(rng, lens, num_blocks, mbps):
    """Block tables [B, mbps] drawing distinct physical blocks for each
    sequence's ceil(len/16) pages from a seeded random permutation."""
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.zeros((len(lens), mbps), np.int32)
    used = 0
    for i, n in enumerate(lens):
        nb = (int(n) + 15) // 16
        assert nb <= mbps and used + nb <= num_blocks
        tables[i, :nb] = perm[used:used + nb]
        used += nb
    return tables
