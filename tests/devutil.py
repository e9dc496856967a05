"""Device-memory plumbing for the GPU tests (torch tensors as buffers).

fp16 data moves as raw binary16 bit patterns: numpy uint16 on the host,
torch.float16 on the device, never through a float conversion."""
import numpy as np
import torch


def to_dev(bits: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)
    return torch.from_numpy(a.copy()).to("cuda").view(torch.float16)


def empty_dev(shape) -> torch.Tensor:
    return torch.empty(shape, dtype=torch.float16, device="cuda")


def to_host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def read_dev(ptr: int, n_elems: int) -> np.ndarray:
    """Copy n_elems fp16 values starting at device address ptr to host bits."""
    import ctypes
    torch.cuda.synchronize()
    out = np.empty(n_elems, dtype=np.uint16)
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rc = hip.hipMemcpy(out.ctypes.data, ptr, 2 * n_elems, 2)  # hipMemcpyDeviceToHost
    assert rc == 0, f"hipMemcpy failed: {rc}"
    return out


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """Normwise max|a-b| / max(|a|,|b|): computeRelativeError of
    tests/test_transformer.cu:80-92.  A non-finite value in one array that the
    other does not hold at the same place gives inf (never NaN, which every
    `<= tol` comparison would let through unnoticed in a max())."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    fa, fb = np.isfinite(a), np.isfinite(b)
    if not (fa.all() and fb.all()):
        same = np.array_equal(fa, fb) and np.array_equal(a[~fa], b[~fb], equal_nan=True)
        if not same:
            return float("inf")
        a, b = a[fa], b[fb]
    mx = max(np.abs(a).max(initial=0.0), np.abs(b).max(initial=0.0))
    return float(np.abs(a - b).max(initial=0.0) / mx) if mx > 0 else 0.0


def to_dev_raw(arr: np.ndarray) -> torch.Tensor:
    """Any numpy array (e.g. int8 weights) to a device tensor of the same bytes."""
    return torch.from_numpy(np.ascontiguousarray(arr).copy()).to("cuda")
