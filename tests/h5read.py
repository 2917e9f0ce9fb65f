"""Read datasets back from an HDF5 file with the HDF5 C library (ctypes), for checking the
monitor file the simulator writes.  Test infrastructure."""
import ctypes as C
import os

import numpy as np

_CANDIDATES = [os.environ.get("HELIOX_HDF5_LIB"), "libhdf5.so", "libhdf5.so.103", "/opt/conda/lib/libhdf5.so",
               "/usr/lib/x86_64-linux-gnu/hdf5/serial/libhdf5.so"]
_lib = None


def lib():
    """The HDF5 C library, or None where it is absent."""
    global _lib
    if _lib is None:
        for name in _CANDIDATES:
            if not name:
                continue
            try:
                _lib = C.CDLL(name)
                break
            except OSError:
                continue
        if _lib is None:
            return None
        L = _lib
        hid = C.c_int64
        L.H5open.restype = C.c_int
        L.H5open()
        L.H5Eset_auto2.argtypes = [hid, C.c_void_p, C.c_void_p]
        L.H5Eset_auto2(0, None, None)
        L.H5Fopen.restype = hid
        L.H5Fopen.argtypes = [C.c_char_p, C.c_uint, hid]
        L.H5Fclose.argtypes = [hid]
        L.H5Dopen2.restype = hid
        L.H5Dopen2.argtypes = [hid, C.c_char_p, hid]
        L.H5Dclose.argtypes = [hid]
        L.H5Dget_space.restype = hid
        L.H5Dget_space.argtypes = [hid]
        L.H5Sclose.argtypes = [hid]
        L.H5Sget_simple_extent_dims.argtypes = [hid, C.POINTER(C.c_ulonglong), C.POINTER(C.c_ulonglong)]
        L.H5Dread.argtypes = [hid, hid, hid, hid, hid, C.c_void_p]
        L.H5Dget_create_plist.restype = hid
        L.H5Dget_create_plist.argtypes = [hid]
        L.H5Pget_chunk.argtypes = [hid, C.c_int, C.POINTER(C.c_ulonglong)]
        L.H5Pclose.argtypes = [hid]
    return _lib


def read_dataset(path, name):
    """(data, maxdim, chunk) of a one-dimensional double dataset; KeyError if absent."""
    L = lib()
    f = L.H5Fopen(path.encode(), 0, 0)            # H5F_ACC_RDONLY, H5P_DEFAULT
    if f < 0:
        raise OSError(f"cannot open {path}")
    try:
        d = L.H5Dopen2(f, name.encode(), 0)
        if d < 0:
            raise KeyError(name)
        try:
            sp = L.H5Dget_space(d)
            dims = (C.c_ulonglong * 1)()
            maxd = (C.c_ulonglong * 1)()
            assert L.H5Sget_simple_extent_dims(sp, dims, maxd) == 1
            L.H5Sclose(sp)
            out = np.empty(int(dims[0]), np.float64)
            native_double = C.c_int64.in_dll(L, "H5T_NATIVE_DOUBLE_g").value
            if out.size:
                assert L.H5Dread(d, native_double, 0, 0, 0, out.ctypes.data_as(C.c_void_p)) >= 0
            pl = L.H5Dget_create_plist(d)
            ch = (C.c_ulonglong * 1)()
            nch = L.H5Pget_chunk(pl, 1, ch)
            L.H5Pclose(pl)
            return out, int(maxd[0]), int(ch[0]) if nch == 1 else None
        finally:
            L.H5Dclose(d)
    finally:
        L.H5Fclose(f)
