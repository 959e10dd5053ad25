"""ctypes binding of libhelrm_hip.so with the interface of Orion's Lattigo
backend (orion/backend/lattigo/bindings.py:104-796): the same method names,
argument conversion (Python lists -> C arrays, floats -> c_float) and
{Data, Length} array results freed through FreeCArray.

Orion selects a backend object in Scheme.setup_backend
(orion/core/orion.py:100-126) and calls `setup_bindings(params)` on it; a
`HipLibrary` is a drop-in for `LattigoLibrary` there.  Errors raise
`HipError` with the library's message instead of aborting the process.
"""
import ctypes

import numpy as np

from . import library_path


class HipError(RuntimeError):
    pass


class ArrayResultInt(ctypes.Structure):
    _fields_ = [("Data", ctypes.POINTER(ctypes.c_int)), ("Length", ctypes.c_ulong)]


class ArrayResultFloat(ctypes.Structure):
    _fields_ = [("Data", ctypes.POINTER(ctypes.c_float)), ("Length", ctypes.c_ulong)]


class ArrayResultUInt64(ctypes.Structure):
    _fields_ = [("Data", ctypes.POINTER(ctypes.c_ulonglong)), ("Length", ctypes.c_ulonglong)]


class ArrayResultByte(ctypes.Structure):
    _fields_ = [("Data", ctypes.POINTER(ctypes.c_char)), ("Length", ctypes.c_ulong)]


_ARRAY_TYPES = (ArrayResultInt, ArrayResultFloat, ArrayResultUInt64)


class HipFunction:
    """Wraps one C entry point: converts arguments as LattigoFunction does
    (orion/backend/lattigo/bindings.py:9-97) and turns the -1 / empty-array
    failure convention into HipError."""

    lib = None

    def __init__(self, func, argtypes, restype, checked=True):
        self.func = func
        self.func.argtypes = argtypes
        self.func.restype = restype
        self.checked = checked

    def __call__(self, *args):
        c_args = []
        for arg in args:
            typ = self.func.argtypes[len(c_args)]
            c_arg = self._to_c(arg, typ)
            if isinstance(c_arg, tuple):
                c_args.extend(c_arg)
            else:
                c_args.append(c_arg)
        res = self.func(*c_args)
        if isinstance(res, ArrayResultByte):
            # as LattigoFunction (bindings.py:86-94): (bytes as uint8, pointer); the caller frees
            # the pointer with FreeCArray, the returned array is a copy and stays valid
            if not res.Data:
                if self.checked and HipFunction.lib is not None:
                    msg = HipFunction.lib.GetLastError().decode()
                    if msg:
                        raise HipError(msg)
                return np.zeros(0, dtype=np.uint8), res.Data
            n = int(res.Length)
            buf = ctypes.cast(res.Data, ctypes.POINTER(ctypes.c_ubyte * n)).contents
            return np.frombuffer(buf, dtype=np.uint8).copy(), res.Data
        if isinstance(res, _ARRAY_TYPES):
            if not res.Data:
                if self.checked and HipFunction.lib is not None:
                    msg = HipFunction.lib.GetLastError().decode()
                    if msg:
                        raise HipError(msg)
                return []
            n = int(res.Length)
            if isinstance(res, ArrayResultFloat):
                out = np.ctypeslib.as_array(res.Data, shape=(n,)).astype(np.float64).tolist()
            else:
                out = [int(res.Data[i]) for i in range(n)]
            HipFunction.lib.FreeCArray(ctypes.cast(res.Data, ctypes.c_void_p))
            return out
        if self.checked and self.func.restype is ctypes.c_int and res == -1:
            raise HipError(HipFunction.lib.GetLastError().decode())
        return res

    @staticmethod
    def _to_c(arg, typ):
        if isinstance(arg, bool):
            return ctypes.c_int(int(arg))
        if isinstance(arg, (int, np.integer)) and typ in (ctypes.c_int, ctypes.c_ulong, ctypes.c_ulonglong, ctypes.c_uint64):
            return typ(int(arg))
        if isinstance(arg, float) and typ is ctypes.c_double:
            return ctypes.c_double(arg)
        if isinstance(arg, float):
            return ctypes.c_float(arg)
        if isinstance(arg, str):
            return arg.encode("utf-8")
        if typ == ctypes.POINTER(ctypes.c_ubyte) and isinstance(arg, (bytes, bytearray, np.ndarray)):
            a = np.ascontiguousarray(np.frombuffer(bytes(arg), dtype=np.uint8) if not isinstance(arg, np.ndarray)
                                     else arg.reshape(-1).view(np.uint8))
            return (a.ctypes.data_as(typ), len(a))
        if isinstance(arg, np.ndarray):
            if typ == ctypes.POINTER(ctypes.c_float):
                a = np.ascontiguousarray(arg, dtype=np.float32)
                return (a.ctypes.data_as(typ), len(a))
            if typ == ctypes.POINTER(ctypes.c_int):
                a = np.ascontiguousarray(arg, dtype=np.int32)
                return (a.ctypes.data_as(typ), len(a))
        if isinstance(arg, (list, tuple)):
            if typ == ctypes.POINTER(ctypes.c_int):
                return ((ctypes.c_int * len(arg))(*arg), len(arg))
            if typ == ctypes.POINTER(ctypes.c_float):
                a = np.ascontiguousarray(np.asarray(arg, dtype=np.float32))
                return (a.ctypes.data_as(typ), len(a))
            if typ == ctypes.POINTER(ctypes.c_uint64):
                return ((ctypes.c_uint64 * len(arg))(*arg), len(arg))
            raise ValueError("unexpected list argument type")
        return arg


_c = ctypes
_I = _c.c_int
_PI = _c.POINTER(_c.c_int)
_PF = _c.POINTER(_c.c_float)
_PU64 = _c.POINTER(_c.c_uint64)
_PB = _c.POINTER(_c.c_ubyte)

# name -> (argtypes, restype); argtypes follow orion/backend/lattigo/bindings.py
_SIGNATURES = {
    # scheme
    "NewScheme": ([_I, _PI, _I, _PI, _I, _I, _I, _c.c_char_p, _c.c_char_p, _c.c_char_p], _I),
    "DeleteScheme": ([], _I),
    "NewSchemeWithModuli": ([_I, _PU64, _I, _PU64, _I, _I, _I, _c.c_uint64], _I),
    "SetSchemeSeed": ([_c.c_uint64], None),
    "GeneratePrimes": ([_I, _PI, _I, _PI, _I, _PU64, _PU64], _I),
    "GetLastError": ([], _c.c_char_p),
    # keys
    "NewKeyGenerator": ([], _I),
    "GenerateSecretKey": ([], _I),
    "GeneratePublicKey": ([], _I),
    "GenerateRelinearizationKey": ([], _I),
    "GenerateEvaluationKeys": ([], _I),
    # encoder
    "NewEncoder": ([], _I),
    "Encode": ([_PF, _I, _I, _c.c_ulong], _I),
    "Decode": ([_I], ArrayResultFloat),
    "DecodeDouble": ([_I, _c.POINTER(_c.c_double), _I], _I),
    # encryptor
    "NewEncryptor": ([], _I),
    "NewDecryptor": ([], _I),
    "Encrypt": ([_I], _I),
    "Decrypt": ([_I], _I),
    "SerializeSecretKey": ([], ArrayResultByte),
    "LoadSecretKey": ([_PB, _c.c_ulong], _I),
    "GenerateAndSerializeRotationKey": ([_I], ArrayResultByte),
    "LoadRotationKey": ([_PB, _c.c_ulong, _c.c_ulong], _I),
    "SerializeDiagonal": ([_I, _I], ArrayResultByte),
    "LoadPlaintextDiagonal": ([_PB, _c.c_ulong, _I, _c.c_ulong], _I),
    "SerializeCiphertext": ([_I], ArrayResultByte),
    "LoadCiphertext": ([_PB, _c.c_ulong], _I),
    "SerializePlaintext": ([_I], ArrayResultByte),
    "LoadPlaintext": ([_PB, _c.c_ulong], _I),
    "RemovePlaintextDiagonals": ([_I], _I),
    "EncodeComplex": ([_PF, _I, _I, _c.c_ulong], _I),
    "DecodeComplex": ([_I], ArrayResultFloat),
    "MulImaginaryUnit": ([_I], _I),
    "MulImaginaryUnitNew": ([_I], _I),
    "LiveHeapBytes": ([], _c.c_ulonglong),
    "StartLiveHeapSampler": ([_I], _I),
    "StopLiveHeapSampler": ([], _c.c_ulonglong),
    "EncryptSeeded": ([_I, _c.c_ulonglong], _I),
    "DropAx": ([_I], _I),
    "ExpandSeededAx": ([_I, _c.c_ulonglong], _I),
    "GetCiphertextBytes": ([_I], _c.c_double),
    "GetCiphertextBxBytes": ([_I], _c.c_double),
    "SetEncryptionCounter": ([_c.c_uint64], _I),
    # evaluator
    "NewEvaluator": ([], _I),
    "AddRotationKey": ([_I], _I),
    "Rotate": ([_I, _I], _I),
    "RotateNew": ([_I, _I], _I),
    "RotateAdd": ([_I, _I], _I),
    "RotateInto": ([_I, _I, _I], _I),
    "Conjugate": ([_I], _I),
    "ConjugateNew": ([_I], _I),
    "Rescale": ([_I], _I),
    "RescaleNew": ([_I], _I),
    "AddPlaintext": ([_I, _I], _I),
    "AddPlaintextNew": ([_I, _I], _I),
    "SubPlaintext": ([_I, _I], _I),
    "SubPlaintextNew": ([_I, _I], _I),
    "AddCiphertext": ([_I, _I], _I),
    "AddCiphertextNew": ([_I, _I], _I),
    "SubCiphertext": ([_I, _I], _I),
    "SubCiphertextNew": ([_I, _I], _I),
    "Negate": ([_I], _I),
    "AddScalar": ([_I, _c.c_float], _I),
    "AddScalarNew": ([_I, _c.c_float], _I),
    "SubScalar": ([_I, _c.c_float], _I),
    "SubScalarNew": ([_I, _c.c_float], _I),
    "MulScalarInt": ([_I, _I], _I),
    "MulScalarIntNew": ([_I, _I], _I),
    "MulScalarFloat": ([_I, _c.c_float], _I),
    "MulScalarFloatNew": ([_I, _c.c_float], _I),
    "MulPlaintext": ([_I, _I], _I),
    "MulPlaintextNew": ([_I, _I], _I),
    "MulRelinCiphertext": ([_I, _I], _I),
    "MulRelinCiphertextNew": ([_I, _I], _I),
    # polynomial evaluator
    "NewPolynomialEvaluator": ([], _I),
    "GenerateMonomial": ([_PF, _I], _I),
    "GenerateChebyshev": ([_PF, _I], _I),
    "EvaluatePolynomial": ([_I, _I, _c.c_ulong], _I),
    # linear transforms
    "NewLinearTransformEvaluator": ([], _I),
    "GenerateLinearTransform": ([_PI, _I, _PF, _I, _I, _c.c_float, _c.c_char_p], _I),
    "EvaluateLinearTransform": ([_I, _I], _I),
    "SetLinearTransformPrerescale": ([_I], _I),
    "GetLinearTransformPrerescale": ([], _I),
    "GetLinearTransformRotationKeys": ([_I], ArrayResultInt),
    "GenerateLinearTransformRotationKey": ([_I], _I),
    "DeleteLinearTransform": ([_I], _I),
    "RemoveRotationKeys": ([], _I),
    # tensors
    "DeletePlaintext": ([_I], _I),
    "DeleteCiphertext": ([_I], _I),
    "GetPlaintextScale": ([_I], _c.c_ulong),
    "GetCiphertextScale": ([_I], _c.c_ulong),
    "GetCiphertextScaleDouble": ([_I], _c.c_double),
    "GetPlaintextScaleDouble": ([_I], _c.c_double),
    "SetPlaintextScale": ([_I, _c.c_ulong], _I),
    "SetCiphertextScale": ([_I, _c.c_ulong], _I),
    "GetPlaintextLevel": ([_I], _I),
    "GetCiphertextLevel": ([_I], _I),
    "GetPlaintextSlots": ([_I], _I),
    "GetCiphertextSlots": ([_I], _I),
    "GetCiphertextDegree": ([_I], _I),
    "GetModuliChain": ([], ArrayResultUInt64),
    "GetAuxModuliChain": ([], ArrayResultUInt64),
    "GetLivePlaintexts": ([], ArrayResultInt),
    "GetLiveCiphertexts": ([], ArrayResultInt),
    "FreeCArray": ([_c.c_void_p], None),
    # raw residues / measurement
    "ExportCiphertext": ([_I, _PU64, _c.c_size_t, _I], _I),
    "ImportCiphertext": ([_PU64, _I, _c.c_double, _I], _I),
    "ExportPlaintext": ([_I, _PU64, _c.c_size_t, _I], _I),
    "ImportPlaintext": ([_PU64, _I, _c.c_double, _I], _I),
    "ExportGaloisKey": ([_c.c_uint64, _PU64, _c.c_size_t], _I),
    "ExportSecretKey": ([_c.POINTER(_c.c_int64), _c.c_size_t], _I),
    "ExportLinearTransformDiagonal": ([_I, _I, _PU64, _c.c_size_t], _I),
    "GetLinearTransformInfo": ([_I, _PI, _I], _I),
    "GetSchemeInfo": ([_PI, _I], _I),
    "Synchronize": ([], _I),
    "SetStream": ([_I], _I),
    "JoinStream": ([_I], _I),
    "DeviceAlloc": ([_c.c_size_t], _c.c_void_p),
    "DeviceFree": ([_c.c_void_p], _I),
    "CopyToDevice": ([_c.c_void_p, _c.c_void_p, _c.c_size_t], _I),
    "CopyToHost": ([_c.c_void_p, _c.c_void_p, _c.c_size_t], _I),
    "NttDevice": ([_c.c_void_p, _I, _I, _I], _I),
    "MulAccDevice": ([_c.c_void_p, _c.c_void_p, _c.c_void_p, _I, _I], _I),
    "GetStream": ([], _c.c_void_p),
    "ValuPeakProbe": ([_c.POINTER(_c.c_double), _I], _I),
    "LaunchProbe": ([_I, _c.POINTER(_c.c_double), _I], _I),
    "KernelTimingEnable": ([_I], _I),
    "KernelTimingGet": ([_c.c_char_p, _c.POINTER(_c.c_long), _c.POINTER(_c.c_double)], _I),
    "GetMemoryStats": ([_PU64, _PU64, _PU64], _I),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib_handle = None


def load_library():
    """dlopen libhelrm_hip.so once (raises if it has not been built)."""
    global _lib_handle
    if _lib_handle is None:
        _lib_handle = ctypes.CDLL(library_path())
        HipFunction.lib = _lib_handle
        _lib_handle.GetLastError.restype = ctypes.c_char_p
        _lib_handle.GetLastError.argtypes = []
        _lib_handle.FreeCArray.argtypes = [ctypes.c_void_p]
        _lib_handle.FreeCArray.restype = None
    return _lib_handle


class DeviceBuffer:
    """A device allocation of uint64 words owned by libhelrm_hip.so."""

    def __init__(self, lib, ptr, shape):
        self.lib, self.ptr, self.shape = lib, ptr, tuple(shape)

    @property
    def nbytes(self):
        return int(np.prod(self.shape)) * 8

    def download(self):
        out = np.empty(self.shape, dtype=np.uint64)
        self.lib.CopyToHost(out.ctypes.data_as(ctypes.c_void_p), self.ptr, self.nbytes)
        return out

    def free(self):
        if self.ptr:
            self.lib.DeviceFree(self.ptr)
            self.ptr = None


class HipLibrary:
    """Drop-in for orion.backend.lattigo.bindings.LattigoLibrary."""

    def __init__(self):
        self.lib = load_library()
        for name, (argtypes, restype) in _SIGNATURES.items():
            setattr(self, name, HipFunction(getattr(self.lib, name), list(argtypes), restype))

    # orion/backend/python/lt_evaluator.py:262-273 reads this flag: False (the
    # default, Lattigo's convention) -- EvaluateLinearTransform returns the
    # un-rescaled result and the caller rescales; True (the convention of the
    # reference's double-hoisted Cheddar path, cheddar/bindings.py:183-187) --
    # the result comes back rescaled, here with the first division fused into
    # the transform's final ModDown and the same residues as the two steps.
    # The flag belongs to the current scheme (a new scheme starts at False).
    @property
    def lt_output_prerescaled(self):
        return self.lib.GetLinearTransformPrerescale() == 1

    def set_lt_output_prerescaled(self, on):
        self.SetLinearTransformPrerescale(1 if on else 0)

    # orion/backend/lattigo/bindings.py:127-138
    def setup_bindings(self, orion_params):
        self.setup_scheme(orion_params)

    # orion/backend/lattigo/bindings.py:140-187
    def setup_scheme(self, orion_params):
        logn = orion_params.get_logn()
        logq = orion_params.get_logq()
        logp = orion_params.get_logp()
        logscale = orion_params.get_logscale()
        h = orion_params.get_hamming_weight()
        ringtype = orion_params.get_ringtype()
        keys_path = orion_params.get_keys_path()
        io_mode = orion_params.get_io_mode()
        seed = getattr(orion_params, "get_seed", lambda: None)()
        if seed is not None:
            self.SetSchemeSeed(int(seed))
        self.NewScheme(logn, list(logq), list(logp), logscale, h, ringtype, keys_path, io_mode)

    # -- helpers for parity checks and benchmarks (numpy views of raw residues)
    def export_ciphertext(self, ct_id, coeff=False):
        level = self.GetCiphertextLevel(ct_id)
        n = 1 << self._logn()
        buf = np.zeros((2, level + 1, n), dtype=np.uint64)
        self.ExportCiphertext(ct_id, buf.ctypes.data_as(_PU64), buf.size, int(coeff))
        return buf

    def import_ciphertext(self, data, level, scale, coeff=False):
        data = np.ascontiguousarray(data, dtype=np.uint64)
        return self.ImportCiphertext(data.ctypes.data_as(_PU64), level, float(scale), int(coeff))

    def export_plaintext(self, pt_id, coeff=False):
        level = self.GetPlaintextLevel(pt_id)
        n = 1 << self._logn()
        buf = np.zeros((level + 1, n), dtype=np.uint64)
        self.ExportPlaintext(pt_id, buf.ctypes.data_as(_PU64), buf.size, int(coeff))
        return buf

    def import_plaintext(self, data, level, scale, coeff=False):
        data = np.ascontiguousarray(data, dtype=np.uint64)
        return self.ImportPlaintext(data.ctypes.data_as(_PU64), level, float(scale), int(coeff))

    def export_galois_key(self, galel):
        L = len(self.GetModuliChain())
        K = len(self.GetAuxModuliChain())
        n = 1 << self._logn()
        dnum = (L + K - 1) // K
        buf = np.zeros((dnum, 2, L + K, n), dtype=np.uint64)
        self.ExportGaloisKey(int(galel), buf.ctypes.data_as(_PU64), buf.size)
        return buf

    def export_secret_key(self):
        n = 1 << self._logn()
        buf = np.zeros(n, dtype=np.int64)
        self.ExportSecretKey(buf.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), n)
        return buf

    def export_lt_diagonal(self, lt_id, diag, level):
        K = len(self.GetAuxModuliChain())
        n = 1 << self._logn()
        buf = np.zeros((level + 1 + K, n), dtype=np.uint64)
        self.ExportLinearTransformDiagonal(lt_id, int(diag), buf.ctypes.data_as(_PU64), buf.size)
        return buf

    def lt_info(self, lt_id):
        out = (ctypes.c_int * 4)()
        self.GetLinearTransformInfo(lt_id, out, 4)
        return {"N1": out[0], "giant": out[1], "baby": out[2], "plaintexts": out[3]}

    def decode_double(self, pt_id):
        n = 1 << (self._logn() - 1)
        buf = np.zeros(n, dtype=np.float64)
        self.DecodeDouble(pt_id, buf.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), n)
        return buf

    # device buffers from the library's allocator (one HIP runtime per process)
    def device_upload(self, arr):
        """Copy a uint64 numpy array to a new device buffer; returns DeviceBuffer."""
        a = np.ascontiguousarray(arr, dtype=np.uint64)
        ptr = self.DeviceAlloc(a.nbytes)
        if not ptr:
            raise HipError(self.GetLastError().decode() or "DeviceAlloc failed")
        buf = DeviceBuffer(self, ptr, a.shape)
        self.CopyToDevice(ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        return buf

    def device_empty(self, shape):
        n = int(np.prod(shape)) * 8
        ptr = self.DeviceAlloc(n)
        if not ptr:
            raise HipError(self.GetLastError().decode() or "DeviceAlloc failed")
        return DeviceBuffer(self, ptr, tuple(shape))

    def kernel_time(self, name):
        cnt = ctypes.c_long(0)
        tot = ctypes.c_double(0.0)
        self.KernelTimingGet(name, ctypes.byref(cnt), ctypes.byref(tot))
        return int(cnt.value), float(tot.value)

    def serialize(self, fn, *args):
        """Bytes of a Serialize* entry point as a numpy uint8 copy (the
        library's buffer is released)."""
        data, ptr = getattr(self, fn)(*args)
        if ptr:
            self.FreeCArray(ptr)
        return data

    def valu_peak(self):
        """Integer VALU issue rate measured on the device (ValuPeakProbe)."""
        out = (ctypes.c_double * 5)()
        self.ValuPeakProbe(out, 5)
        return {"wave_instr_per_s": out[0], "cus": int(out[1]), "wave_instr_per_clk_per_cu": out[2],
                "v_mad_u64_u32_per_s": out[3], "v_add3_u32_per_s": out[4]}

    def launch_probe(self, limbs):
        """Dependent-launch latency and the copy time of `limbs` rows (LaunchProbe)."""
        out = (ctypes.c_double * 3)()
        self.LaunchProbe(limbs, out, 3)
        return {"empty_launch_us": out[0], "copy_us": out[1], "copy_TBs": out[2]}

    def memory_stats(self):
        a, b, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        self.GetMemoryStats(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
        return {"live": a.value, "cached": b.value, "peak": c.value}

    def scheme_info(self):
        out = (ctypes.c_int * 6)()
        self.GetSchemeInfo(out, 6)
        return {"logN": out[0], "L": out[1], "K": out[2], "dnum": out[3], "logscale": out[4], "h": out[5]}

    def _logn(self):
        return self.scheme_info()["logN"]
