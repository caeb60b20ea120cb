"""MappedHostVPool -- pinned, device-mapped host V pool (mem-v tier).

Same layout and role as the reference ``tier/pool.py:104-151``: (L, NB, n_kv, page, d) in
host DRAM, keyed by physical block, so the (layer, block, kv-head) page at element offset
((l*NB + blk)*n_kv + kv)*page*d is contiguous.  Allocated with
``amass_host_pool_alloc`` = hipHostMalloc(hipHostMallocMapped) + hipHostGetDevicePointer,
so kernels read it directly over the host link (zero copy) and the copy engine can DMA
from it.  ``host`` is a CPU torch view of the same bytes (for writes / tests);
``dev_ptr`` is the device address kernels take.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from .._hip import AmassError, check, load_library

_ELEM = {torch.bfloat16: 2, torch.float16: 2}


class MappedHostVPool:
    def __init__(self, *, num_layers: int, num_blocks: int, n_kv: int, page: int, d: int,
                 dtype: torch.dtype = torch.bfloat16, device=None, max_pool_gb: float = 256.0):
        if dtype not in _ELEM:
            raise ValueError(f"pool dtype must be bf16/fp16, got {dtype}")
        self.L, self.NB, self.n_kv, self.page, self.d, self.dtype = (
            num_layers, num_blocks, n_kv, page, d, dtype)
        n = num_layers * num_blocks * n_kv * page * d
        nbytes = n * _ELEM[dtype]
        if nbytes > max_pool_gb * (1 << 30):
            raise AmassError(f"pinned V pool would be {nbytes / 2**30:.1f} GiB "
                             f"(> max_pool_gb={max_pool_gb})")
        lib = load_library()
        h, dptr = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib.amass_host_pool_alloc(nbytes, ctypes.byref(h), ctypes.byref(dptr)),
              "amass_host_pool_alloc")
        self._host_ptr = h.value
        self.dev_ptr = dptr.value
        buf = (ctypes.c_int16 * n).from_address(self._host_ptr)
        arr = np.ctypeslib.as_array(buf)
        self.host = torch.from_numpy(arr).view(dtype).view(num_layers, num_blocks, n_kv, page, d)
        self.host.zero_()
        self.pool_gib = nbytes / 2**30
        self.device = device

    def page_offset(self, layer: int, blk: int, kv: int) -> int:
        """Element offset of the (layer, block, kv-head) page."""
        return ((layer * self.NB + blk) * self.n_kv + kv) * self.page * self.d

    def write_layer(self, layer: int, v_blocks: torch.Tensor) -> None:
        """Copy a layer's V (NB, page, n_kv, d) (any device) into the pool layout."""
        self.host[layer].copy_(v_blocks.permute(0, 2, 1, 3).to("cpu"))

    def close(self) -> None:
        if getattr(self, "_host_ptr", None):
            self.host = None
            load_library().amass_host_pool_free(ctypes.c_void_p(self._host_ptr))
            self._host_ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    def vram_note(self) -> str:
        return (f"host_pool={self.pool_gib:.2f}GiB (DRAM, keyed by NB={self.NB}; VRAM hot "
                "buffer bounded to the working set)")
