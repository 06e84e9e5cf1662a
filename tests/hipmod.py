"""Minimal ctypes access to HIP's module API for test-only code objects
(kernels the runtime does not load, e.g. the MFMA layout probes).  Memory
and streams come from torch."""
import ctypes

_hip = None


def _lib():
    global _hip
    if _hip is None:
        # by soname: reuse the HIP runtime already loaded by torch/libbwpp_hip
        _hip = ctypes.CDLL("libamdhip64.so.7")
    return _hip


class Module:
    def __init__(self, path):
        self.mod = ctypes.c_void_p()
        rc = _lib().hipModuleLoad(ctypes.byref(self.mod), path.encode())
        if rc != 0:
            raise RuntimeError(f"hipModuleLoad({path}) failed: {rc}")

    def function(self, name):
        f = ctypes.c_void_p()
        rc = _lib().hipModuleGetFunction(ctypes.byref(f), self.mod, name.encode())
        if rc != 0:
            raise RuntimeError(f"hipModuleGetFunction({name}) failed: {rc}")
        return f

    def launch(self, name, grid, block, args: ctypes.Structure, stream=0, shmem=0):
        f = self.function(name)
        params = (ctypes.c_void_p * 1)(ctypes.addressof(args))
        lib = _lib()
        lib.hipModuleLaunchKernel.argtypes = [ctypes.c_void_p] + [ctypes.c_uint] * 6 + [
            ctypes.c_uint, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        rc = lib.hipModuleLaunchKernel(f, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                       shmem, ctypes.c_void_p(stream), params, None)
        if rc != 0:
            raise RuntimeError(f"hipModuleLaunchKernel({name}) failed: {rc}")

    def close(self):
        if self.mod:
            _lib().hipModuleUnload(self.mod)
            self.mod = None
