"""Building-scale field step on the device (the sbx_fdm_* entry points of
libsbenv.so): the reference core's sb_fdm_step_batch
(complete_port/csim/sb_fdm.h:60-68) for G envs that share one blob's baked
factorization. Inputs live in device memory (torch tensors); the field state
stays on the device between steps.

    f = FieldGroup(blob, n_envs)
    f.step(input_q, ambient, h, air_g, air_T)   # torch float64 cuda tensors
    temp, mass = f.state()                        # host copies, env-major

input_q is (G, n_cvs), ambient and h are (G,), air_g and air_T are (G, k)
(env-major, as the reference's per-env arguments).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import env as E

P = ctypes.c_void_p


class SbxFdmInfo(ctypes.Structure):
    _fields_ = [("n_cvs", ctypes.c_int), ("n_solved", ctypes.c_int), ("k", ctypes.c_int),
                ("n_envs", ctypes.c_int), ("envs_per_block", ctypes.c_int), ("n_blocks", ctypes.c_int),
                ("levels_l", ctypes.c_int), ("levels_u", ctypes.c_int),
                ("nnz_l", ctypes.c_longlong), ("nnz_u", ctypes.c_longlong),
                ("bytes_per_step", ctypes.c_double), ("flops_per_step", ctypes.c_double),
                ("tail_rows_l", ctypes.c_int), ("tail_rows_u", ctypes.c_int),
                ("tail_levels_l", ctypes.c_int), ("tail_levels_u", ctypes.c_int),
                ("chunked_levels_l", ctypes.c_int), ("chunked_levels_u", ctypes.c_int)]

EXACT = 1   # SBX_FDM_EXACT: every level in the reference's order, bit-identical results


_BOUND = False


def _lib() -> ctypes.CDLL:
    global _BOUND
    L = E.lib()
    if not _BOUND:
        L.sbx_fdm_open.restype = P
        L.sbx_fdm_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.sbx_fdm_close.argtypes = [P]
        L.sbx_fdm_info.argtypes = [P, ctypes.POINTER(SbxFdmInfo)]
        L.sbx_fdm_step.argtypes = [P, P, P, P, P, P, P]
        L.sbx_fdm_reset.argtypes = [P, P]
        L.sbx_fdm_get_state.argtypes = [P, P, P]
        L.sbx_fdm_set_state.argtypes = [P, P, P]
        L.sbx_fdm_sensed_response.argtypes = [P, P]
        L.sbx_fdm_air_responses.argtypes = [P, P]
        L.sbx_fdm_lu_solve.argtypes = [P, P, P, ctypes.c_int]
        for f in (L.sbx_fdm_info, L.sbx_fdm_step, L.sbx_fdm_reset, L.sbx_fdm_get_state, L.sbx_fdm_set_state,
                  L.sbx_fdm_sensed_response, L.sbx_fdm_air_responses, L.sbx_fdm_lu_solve):
            f.restype = ctypes.c_int
        _BOUND = True
    return L


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(P)


class FieldGroup:
    def __init__(self, blob: str | Path, n_envs: int, envs_per_block: int = 0, exact: bool = False):
        import torch

        torch.cuda.init()   # torch's HIP runtime state before the library's first HIP call
        L = _lib()
        self.L = L
        self.h = L.sbx_fdm_open(str(blob).encode(), int(n_envs), int(envs_per_block), EXACT if exact else 0)
        if not self.h:
            raise RuntimeError(f"sbx_fdm_open: {L.sbx_last_error().decode()}")
        info = SbxFdmInfo()
        L.sbx_fdm_info(self.h, ctypes.byref(info))
        self.info = info
        self.G, self.n_cvs, self.n, self.k = info.n_envs, info.n_cvs, info.n_solved, info.k

    def close(self):
        if getattr(self, "h", None):
            self.L.sbx_fdm_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int, what: str):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.L.sbx_last_error().decode()}")

    def step(self, input_q, ambient, h, air_g, air_T, stream=None):
        """One step of every env; arguments are float64 cuda tensors (see module doc)."""
        import torch

        G, k = self.G, self.k
        args = [(input_q, (G, self.n_cvs)), (ambient, (G,)), (h, (G,)), (air_g, (G, k)), (air_T, (G, k))]
        for t, shape in args:
            if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float64 and t.is_contiguous()
                    and tuple(t.shape) == shape):
                raise ValueError(f"expected a contiguous float64 cuda tensor of shape {shape}")
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        self._check(self.L.sbx_fdm_step(self.h, *(P(t.data_ptr()) for t, _ in args), P(s)), "sbx_fdm_step")

    def reset(self, stream=None):
        import torch

        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        self._check(self.L.sbx_fdm_reset(self.h, P(s)), "sbx_fdm_reset")

    def state(self) -> tuple[np.ndarray, np.ndarray]:
        T = np.zeros((self.G, self.n_cvs))
        M = np.zeros((self.G, self.n))
        self._check(self.L.sbx_fdm_get_state(self.h, _ptr(T), _ptr(M)), "sbx_fdm_get_state")
        return T, M

    def set_state(self, T: np.ndarray, M: np.ndarray):
        T = np.ascontiguousarray(T, np.float64)
        M = np.ascontiguousarray(M, np.float64)
        assert T.shape == (self.G, self.n_cvs) and M.shape == (self.G, self.n)
        self._check(self.L.sbx_fdm_set_state(self.h, _ptr(T), _ptr(M)), "sbx_fdm_set_state")

    def sensed_response(self) -> np.ndarray:
        S = np.zeros((self.k, self.k))
        self._check(self.L.sbx_fdm_sensed_response(self.h, _ptr(S)), "sbx_fdm_sensed_response")
        return S

    def air_responses(self) -> np.ndarray | None:
        """R [k][n_solved] of the default mode (None in exact mode or without an air side)."""
        R = np.zeros((self.k, self.info.n_solved))
        rc = self.L.sbx_fdm_air_responses(self.h, _ptr(R))
        if rc == 1:
            return None
        self._check(rc, "sbx_fdm_air_responses")
        return R

    def lu_solve(self, b: np.ndarray) -> np.ndarray:
        b = np.ascontiguousarray(np.atleast_2d(b), np.float64)
        x = np.zeros_like(b)
        self._check(self.L.sbx_fdm_lu_solve(self.h, _ptr(b), _ptr(x), b.shape[0]), "sbx_fdm_lu_solve")
        return x
