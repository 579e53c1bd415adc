"""Exact-size, device-mapped pinned host memory for the tier's host store.

Mirrors lazykv/pinned.py: `pinned_empty(shape, dtype)` (:31-42) returns a page-locked CPU tensor of
exactly its size that is released when collected, and `device_view(t)` (:73-92) returns a device
tensor aliasing it, so kernels that read the view read host RAM over PCIe in place.

The reference page-locks an ordinary allocation with cudaHostRegister. Here the pool is allocated
pinned and mapped from the start (`lkv_host_alloc`, hipHostMalloc with the mapped flag): the same
exact size, no caching allocator, no registration step. Coarse-grained memory is the default
(the device may cache it within a kernel; the host pool is written between kernels only);
`coherent=True` asks for fine-grained memory instead.
"""

from __future__ import annotations

import bisect
import ctypes
import threading
import weakref

import torch

from lazykv_amd import _lib

# Live allocations: sorted host base addresses -> (nbytes, device base address). Finalizers may
# run on any thread, so every read and update holds the lock.
_BASES: list[int] = []
_ALLOCS: dict[int, tuple[int, int]] = {}
_LOCK = threading.Lock()


def _free(ptr: int) -> None:
    with _LOCK:
        i = bisect.bisect_left(_BASES, ptr)
        if i < len(_BASES) and _BASES[i] == ptr:
            _BASES.pop(i)
            _ALLOCS.pop(ptr, None)
    try:
        _lib.lib().lkv_host_free(ptr)
    except Exception:  # noqa: BLE001 -- at interpreter exit the runtime may already be gone
        pass


def pinned_empty(shape: tuple[int, ...], dtype: torch.dtype, coherent: bool = False) -> torch.Tensor:
    """An uninitialised CPU tensor in mapped pinned memory, exactly its size, freed when collected."""
    numel = 1
    for s in shape:
        numel *= int(s)
    nbytes = numel * torch.empty((), dtype=dtype).element_size()
    if nbytes == 0:
        return torch.empty(shape, dtype=dtype)
    torch.cuda.init()
    ptr = ctypes.c_void_p()
    _lib.check(_lib.lib().lkv_host_alloc(nbytes, _lib.HOST_COHERENT if coherent else 0, ctypes.byref(ptr)), f"pinning {nbytes} bytes")
    host = int(ptr.value)
    dev = ctypes.c_void_p()
    _lib.check(_lib.lib().lkv_host_device_pointer(host, ctypes.byref(dev)), "device address of the host pool")
    buf = (ctypes.c_uint8 * nbytes).from_address(host)
    t = torch.frombuffer(buf, dtype=torch.uint8, count=nbytes).view(dtype).view(shape)
    with _LOCK:
        bisect.insort(_BASES, host)
        _ALLOCS[host] = (nbytes, int(dev.value))
    # Tied to the buffer object, which the tensor's storage (shared by every view) keeps alive:
    # the memory is released only when the last view is gone.
    weakref.finalize(buf, _free, host)
    return t


def device_address(t: torch.Tensor) -> int:
    """The device address of the first element of a CPU tensor that lives in a pinned_empty pool."""
    ptr = t.data_ptr()
    with _LOCK:
        i = bisect.bisect_right(_BASES, ptr) - 1
        if i >= 0:
            base = _BASES[i]
            nbytes, dev = _ALLOCS[base]
            if ptr < base + nbytes:
                return dev + (ptr - base)
    raise ValueError("tensor is not in memory from pinned_empty; the device cannot read it in place")


def is_mapped(t: torch.Tensor) -> bool:
    try:
        device_address(t)
    except ValueError:
        return False
    return True


class _DeviceArray:
    """The minimal `__cuda_array_interface__` torch.as_tensor needs to wrap a device pointer."""

    def __init__(self, ptr: int, nbytes: int) -> None:
        self.__cuda_array_interface__ = {"shape": (nbytes,), "typestr": "|u1", "data": (ptr, False), "version": 3, "strides": None}


def device_view(t: torch.Tensor) -> torch.Tensor:
    """A device tensor aliasing the pinned CPU tensor `t`: kernels reading it read host RAM over PCIe.

    Reads are zero-copy: no transfer is launched. The caller keeps `t` alive for as long as the view.
    """
    if not t.is_contiguous():
        raise ValueError("device_view needs a contiguous pinned tensor")
    ptr = device_address(t)
    nbytes = t.numel() * t.element_size()
    raw = torch.as_tensor(_DeviceArray(ptr, nbytes), device="cuda")
    return raw.view(t.dtype).view(t.shape)
