"""ctypes binding of the `.oil` reader in libmythos_host.so
(include/mythos_oil_file.h).

`OILReader` keeps the reference's reader vocabulary (src/oil_format.cpp:287-462:
valid(), tensor_names(), read_config()) but hands tensors out quantised, in
the structure-of-arrays layouts the kernels of libmythos_oil.so take:

    repack(name, rows, cols)  -> host numpy arrays (indices, codebooks, cb_block)
    upload(name, rows, cols)  -> torch device tensors, same layouts

so a model file feeds mythos_oil.oil4_gemv / oil8_gemv / i2s_gemv_f32 without an
FP32 copy of its weights.  Errors raise MythosError with the library's message.
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

import mythos_oil  # loads torch, then libmythos_oil.so, which libmythos_host.so links

HOST_LIB_PATH = mythos_oil.HOST_LIB_PATH

# Every extern "C" symbol declared in include/mythos_oil_file.h.
EXPORTS = (
    "mth_oil_open", "mth_oil_close", "mth_oil_error",
    "mth_oil_num_tensors", "mth_oil_tensor_name", "mth_oil_tensor_info",
    "mth_oil_repack", "mth_oil_upload",
)

OK, EINVAL, EFORMAT, EUNSUPPORTED, EDEVICE = 0, -1, -2, -3, -4
BINARY, TERNARY, OIL4, OIL8, FP32 = 0, 1, 2, 3, 5

_lib = mythos_oil.load_library(HOST_LIB_PATH)
VP, I64, I32 = C.c_void_p, C.c_int64, C.c_int
P64 = C.POINTER(C.c_int64)
_lib.mth_oil_open.argtypes = [C.c_char_p]
_lib.mth_oil_open.restype = VP
_lib.mth_oil_close.argtypes = [VP]
_lib.mth_oil_close.restype = None
_lib.mth_oil_error.argtypes = []
_lib.mth_oil_error.restype = C.c_char_p
_lib.mth_oil_num_tensors.argtypes = [VP]
_lib.mth_oil_num_tensors.restype = I64
_lib.mth_oil_tensor_name.argtypes = [VP, I64]
_lib.mth_oil_tensor_name.restype = C.c_char_p
_lib.mth_oil_tensor_info.argtypes = [VP, C.c_char_p, C.POINTER(I32), P64, P64, P64]
_lib.mth_oil_tensor_info.restype = I32
_lib.mth_oil_repack.argtypes = [VP, C.c_char_p, I64, I64, I32, VP, I64, VP, I64, P64]
_lib.mth_oil_repack.restype = I32
_lib.mth_oil_upload.argtypes = [VP, C.c_char_p, I64, I64, I32, VP, I64, VP, I64, P64, VP]
_lib.mth_oil_upload.restype = I32
lib = _lib


def last_error() -> str:
    return _lib.mth_oil_error().decode()


def _check(rc: int) -> None:
    if rc != OK:
        raise mythos_oil.MythosError(rc, last_error())


def layout_bytes(fmt: int, rows: int, cols: int, num_blocks: int, in_major: bool = False) -> tuple[int, int]:
    """(index bytes, codebook bytes) of a rows x cols tensor in the kernels'
    layout: OIL4 nibbles + 16 FP16 per block (one codebook when input-major),
    OIL8 bytes + 256 FP32, ternary 2-bit codes + 3 FP32, FP32 floats."""
    n = rows * cols
    if fmt == OIL4:
        return (n + 1) // 2, 32 * (1 if in_major else num_blocks)
    if fmt == OIL8:
        return n, 1024
    if fmt == TERNARY:
        return (n + 3) // 4, 12
    return 4 * n, 0


class OILReader:
    """An open `.oil` file (memory-mapped, indexed once)."""

    def __init__(self, path: str):
        self.path = os.fspath(path)
        self._h = _lib.mth_oil_open(self.path.encode())
        self.error = "" if self._h else last_error()

    def valid(self) -> bool:
        return bool(self._h)

    def _need(self):
        if not self._h:
            raise mythos_oil.MythosError(EFORMAT, self.error or "file not open")
        return self._h

    def close(self) -> None:
        if self._h:
            _lib.mth_oil_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()

    def read_config(self) -> bytes:
        """The header's config bytes (OILReader::read_config)."""
        with open(self.path, "rb") as f:
            head = f.read(16)
            (size,) = struct.unpack_from("<I", head, 12)
            return f.read(size)

    def tensor_names(self) -> list[str]:
        h = self._need()
        return [_lib.mth_oil_tensor_name(h, i).decode() for i in range(_lib.mth_oil_num_tensors(h))]

    def info(self, name: str) -> dict:
        fmt, nw, nb, bw = I32(), I64(), I64(), I64()
        _check(_lib.mth_oil_tensor_info(self._need(), name.encode(), C.byref(fmt), C.byref(nw), C.byref(nb),
                                        C.byref(bw)))
        return {"format": fmt.value, "num_weights": nw.value, "num_blocks": nb.value,
                "block_weights": bw.value}

    def repack(self, name: str, rows: int, cols: int, in_major: bool = False):
        """Host copy in the kernels' layout: (indices u8, codebooks, cb_block),
        rows = output features.  codebooks is u16 FP16 bits [blocks][16] for
        OIL4, f32[256] for OIL8, f32[3] for ternary, None for FP32 (indices
        then hold the floats).  in_major: the file holds the weight as the
        reference's Linear does, element (m, k) at k*rows + m."""
        inf = self.info(name)
        ib, cbb = layout_bytes(inf["format"], rows, cols, inf["num_blocks"], in_major)
        idx = np.zeros(max(ib, 1), np.uint8)
        cbs = np.zeros(max(cbb, 4), np.uint8)
        cbk = I64(0)
        _check(_lib.mth_oil_repack(self._need(), name.encode(), rows, cols, int(in_major), idx.ctypes.data, ib,
                                   cbs.ctypes.data if cbb else None, cbb, C.byref(cbk)))
        idx = idx[:ib]
        fmt = inf["format"]
        if fmt == OIL4:
            return idx.reshape(rows, cols // 2), cbs[:cbb].view(np.uint16).reshape(-1, 16), cbk.value
        if fmt == OIL8:
            return idx.reshape(rows, cols), cbs[:cbb].view(np.float32), 0
        if fmt == TERNARY:
            return idx, cbs[:12].view(np.float32), 0
        return idx.view(np.float32).reshape(rows, cols), None, 0

    def upload(self, name: str, rows: int, cols: int, device="cuda", stream=None, in_major: bool = False):
        """Device tensors (indices, codebooks, cb_block) in the kernels'
        layout, copied on `stream` (torch's current stream by default)."""
        torch = mythos_oil._torch()
        inf = self.info(name)
        fmt = inf["format"]
        ib, cbb = layout_bytes(fmt, rows, cols, inf["num_blocks"], in_major)
        idx = torch.empty(ib, dtype=torch.uint8, device=device)
        cbs = torch.empty(max(cbb, 1), dtype=torch.uint8, device=device)
        cbk = I64(0)
        _check(_lib.mth_oil_upload(self._need(), name.encode(), rows, cols, int(in_major), idx.data_ptr(), ib,
                                   cbs.data_ptr() if cbb else None, cbb, C.byref(cbk),
                                   mythos_oil._stream(stream)))
        if fmt == OIL4:
            return idx.view(rows, cols // 2), cbs.view(torch.int16), cbk.value
        if fmt == OIL8:
            return idx.view(rows, cols), cbs.view(torch.float32), 0
        if fmt == TERNARY:
            return idx, cbs[:12].view(torch.float32), 0
        return idx.view(torch.float32).view(rows, cols), None, 0
