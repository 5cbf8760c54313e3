"""Grouped decode GEMV: several E8-packed linears in one HIP launch.

The decode path of a decoder layer runs q/k/v (and gate/up) on the same
activations; the reference runs one unpack + dense GEMM per linear
(``_FusedE8GEMMFunction.forward``, ``ojasx2/math/lattice.py:610-624``).
``GroupedGemv`` plans a table of linears once (``ojx_e8t_gemv_grouped_plan``)
and launches them together (``ojx_e8t_gemv_grouped``).  Each job computes
exactly what ``ops.e8t_linear`` computes for it.

Typical uses:

* fused projections -- ``GroupedGemv.fused(layers, M, dtype)``: the outputs of
  the layers are concatenated along the last dim of one ``[M, sum(N)]`` tensor
  and every job reads the launch's ``x`` (at most 4 jobs travel in the kernel
  arguments, no device table); layers with a LoRA adapter get it fused: the grouped
  launch first computes u = scaling * x @ A for all adapters (one launch), and the
  GEMV adds u @ B in its epilogue (E8LatticeLinear.forward, lattice.py:839-842).  The
  plan holds the adapter tensors themselves (lora_A / lora_B must already be
  contiguous in the activation dtype), so in-place updates of them are seen; a new
  scaling needs a new plan.  Such a plan also owns one fp32 u buffer per adapter, which
  every call writes and then reads: unless the launch forms u inside the GEMV (rank-8
  adapters on the single-round staged-tile route), calls of one plan that overlap (two
  streams, or graph replays that are not ordered on one stream) race on it, so use such a
  plan from one stream at a time (or build one plan per stream);
* a fixed table -- explicit ``x`` / ``y`` per job, uploaded once to the device.

Ternary (bitrate 1.5) groups take group size 32 (``ojx_e8t_gemv_grouped``); 2-bit groups
(bitrate 2.0, ``E8LatticePacker``, the reference's default) and 1-bit groups (bitrate 1.0,
``RootE8LatticePacker``) take group size 8, 16, 32 or 64, one per group
(``ojx_e8_gemv_grouped``, ``ojx_e8r_gemv_grouped``).
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import torch

from . import _native as N
from . import ops


def _job(packed: torch.Tensor, scales: torch.Tensor, bias: Optional[torch.Tensor], n: int,
         k: int, x: Optional[torch.Tensor] = None, y: Optional[torch.Tensor] = None,
         y_col: int = 0, y_ld: int = 0) -> N.GemvJob:
    j = N.GemvJob()  # zero-initialised: no LoRA adapter
    j.x = N.ptr(x)
    j.packed = packed.data_ptr()
    j.scales = scales.data_ptr()
    j.bias = N.ptr(bias)
    j.y = N.ptr(y)
    j.N, j.K, j.y_col, j.y_ld, j.wg_begin = n, k, y_col, y_ld, 0
    return j


class GroupedGemv:
    """A planned group of decode-GEMV jobs for batch ``M`` and activation ``dtype``."""

    def __init__(self, jobs: Sequence[N.GemvJob], M: int, dtype: torch.dtype,
                 device: torch.device, keep: Sequence[torch.Tensor] = (), bitrate: float = 1.5,
                 group_size: int = 32) -> None:
        if dtype not in (torch.bfloat16, torch.float16):
            raise RuntimeError("grouped GEMV takes bfloat16 or float16 activations")
        if float(bitrate) not in (1.0, 1.5, 2.0):
            raise RuntimeError("grouped GEMV runs ternary (1.5), 2-bit (2.0) or 1-bit (1.0) "
                               "linears")
        self.bitrate = float(bitrate)
        self.group_size = int(group_size)
        if self.bitrate == 1.5 and self.group_size != 32:
            raise RuntimeError("grouped ternary GEMV needs group_size 32")
        self.M = int(M)
        self.dtype = dtype
        self.device = torch.device(device)
        self.n = len(jobs)
        # Workgroups start in job order; a job's workgroups run K / 1024 rounds each, so the
        # longest-K jobs go first and the launch does not end on a tail of long workgroups
        # (224-linear stack, M = 1: 439 -> 378 us).  Every job keeps its own output place.
        jobs = sorted(jobs, key=lambda j: -int(j.K))
        self._arr = (N.GemvJob * self.n)(*jobs)
        grid = ctypes.c_int64(0)
        if self.bitrate == 1.5:
            N.check(N.lib().ojx_e8t_gemv_grouped_plan(ctypes.addressof(self._arr), self.n,
                                                      self.M, N.DTYPE_CODE[dtype],
                                                      ctypes.byref(grid)), "gemv_grouped_plan")
        else:
            plan = (N.lib().ojx_e8_gemv_grouped_plan if self.bitrate == 2.0
                    else N.lib().ojx_e8r_gemv_grouped_plan)
            N.check(plan(ctypes.addressof(self._arr), self.n, self.M, self.group_size,
                         N.DTYPE_CODE[dtype], ctypes.byref(grid)), "e8/e8r gemv_grouped_plan")
        self.grid = grid.value
        self._keep = list(keep)  # tensors the job pointers refer to
        self._lora = []          # layers whose adapter is fused (A, B, scaling read at plan time)
        self._dev = None
        if self.n > 4:
            raw = bytes(ctypes.string_at(ctypes.addressof(self._arr), ctypes.sizeof(self._arr)))
            self._dev = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.device)

    @classmethod
    def fused(cls, layers: Sequence[torch.nn.Module], M: int, dtype: torch.dtype
              ) -> "GroupedGemv":
        """Jobs for E8LatticeLinear-like layers (packed_weight, block_scales, bias,
        out_features, in_features; rank, lora_A, lora_B, scaling for adapters) whose outputs
        are concatenated along dim -1."""
        n_total = sum(int(l.out_features) for l in layers)
        jobs, col, keep, lora = [], 0, [], []
        dev = layers[0].packed_weight.device
        bitrate = float(getattr(layers[0], "bitrate", 1.5))
        gs = int(layers[0].group_size)
        for l in layers:
            if float(getattr(l, "bitrate", 1.5)) != bitrate or int(l.group_size) != gs:
                raise RuntimeError("grouped GEMV: every layer needs the same bitrate and "
                                   "group_size")
            bias = l.bias.detach().to(dtype).contiguous() if l.bias is not None else None
            if bias is not None:
                keep.append(bias)
            # fp16 scale bits; a module cast (.to(bfloat16)) leaves the buffer in another dtype
            scales = l.block_scales.detach().to(torch.float16).contiguous()
            j = _job(l.packed_weight, scales, bias, int(l.out_features),
                     int(l.in_features), y_col=col, y_ld=n_total)
            if getattr(l, "rank", 0) > 0 and getattr(l, "lora_A", None) is not None:
                if getattr(l, "use_hadamard", False):
                    raise RuntimeError("grouped GEMV: adapters of Hadamard-rotated layers are "
                                       "not fused")
                for name in ("lora_A", "lora_B"):
                    t = getattr(l, name)
                    if t.dtype != dtype or not t.is_contiguous():
                        raise RuntimeError(f"grouped GEMV: {name} must be contiguous in the "
                                           "activation dtype")
                r = int(l.lora_A.shape[-1])
                if not 1 <= r <= ops.LORA_MAX_RANK:
                    raise RuntimeError(f"grouped GEMV: LoRA rank {r} out of range")
                u = torch.empty((int(M), r), dtype=torch.float32, device=dev)
                j.lora_u, j.lora_b, j.lora_r, j.lora_ldu = u.data_ptr(), l.lora_B.data_ptr(), r, r
                j.lora_a, j.lora_scaling = l.lora_A.data_ptr(), float(l.scaling)
                keep += [u, l.lora_A, l.lora_B]
                lora.append(l)
            jobs.append(j)
            keep += [l.packed_weight, scales]
            col += int(l.out_features)
        g = cls(jobs, M, dtype, dev, keep, bitrate=bitrate, group_size=gs)
        g.n_total = n_total
        g._lora = lora
        return g

    def __call__(self, x: Optional[torch.Tensor] = None, y: Optional[torch.Tensor] = None,
                 stream: Optional[torch.cuda.Stream] = None) -> Optional[torch.Tensor]:
        if x is not None:
            if x.dtype != self.dtype or not x.is_contiguous():
                raise RuntimeError("x must be contiguous and of the planned dtype")
            if x.numel() // x.shape[-1] != self.M:
                raise RuntimeError(f"x has {x.numel() // x.shape[-1]} rows, planned for {self.M}")
        if y is None and hasattr(self, "n_total") and x is not None:
            y = torch.empty((*x.shape[:-1], self.n_total), dtype=self.dtype, device=self.device)
        s = stream.cuda_stream if stream is not None else N.stream_handle(self.device)
        if self.bitrate == 1.5:
            N.check(N.lib().ojx_e8t_gemv_grouped(ctypes.addressof(self._arr),
                                                 N.ptr(self._dev), self.n, N.ptr(x), N.ptr(y),
                                                 self.M, N.DTYPE_CODE[self.dtype], s),
                    "gemv_grouped")
        else:
            launch = (N.lib().ojx_e8_gemv_grouped if self.bitrate == 2.0
                      else N.lib().ojx_e8r_gemv_grouped)
            N.check(launch(ctypes.addressof(self._arr), N.ptr(self._dev), self.n, N.ptr(x),
                           N.ptr(y), self.M, self.group_size, N.DTYPE_CODE[self.dtype], s),
                    "e8/e8r gemv_grouped")
        return y


def stack_jobs(linears: Sequence[dict], xs: dict, ys: List[torch.Tensor]) -> List[N.GemvJob]:
    """Jobs with explicit x and y for a table of {packed, scales, N, K} dicts."""
    return [_job(l["packed"], l["scales"], None, l["N"], l["K"], x=xs[l["K"]], y=y)
            for l, y in zip(linears, ys)]
