"""PyTorch operators over the C ABI of libsffft.so.

The reference names a library with a PyTorch binding as its next step (README.md:177), for the
long-convolution layers of Hyena/H3/S4-style models (README.md:11). This module provides it:

- ``torch.ops.sffft.spectrum(k, plan, conj=False)``: the kernel-order spectrum [H, 2L]
  complex64 of a real filter k [H, L] (fp32), or its conjugate;
- ``torch.ops.sffft.conv(u, kf, plan)``: y = causal_conv(u, k) for u [B, H, L] fp32 or bf16;
- ``LongConv``: the two together, with the spectrum cached per (filter tensor, its version, L,
  plan), so a layer whose filter does not change computes the spectrum once.

``plan`` is the list of the nine ``sffft_plan`` fields (``plan_fields``). The operators, their GPU
kernels and their autograd are registered from C++ (``csrc/torch_ops.cpp``, built into
``libsffft_torch.so``), so a call costs the dispatcher's few microseconds rather than the
Python wrappers of ``torch.library.custom_op``. Their fake (meta) implementations are here, so
they trace under ``torch.compile`` and ``torch.export``; they launch on the current stream, so
they capture into CUDA/HIP graphs.

Gradients:

- ``conv`` is differentiable in u. Causal convolution's adjoint is the anti-causal correlation
  du[m] = sum_{n >= m} dy[n] k[n - m]. With the N = 2L zero padding this is
  IDFT(DFT(dy) * conj(K))[m] for m < L, so the backward pass runs the same kernel on the
  conjugated spectrum (elementwise conjugation of the kernel-order buffer), with no time
  reversal.
- ``LongConv`` is differentiable in u and in the filter k. The filter gradient is the
  batch-summed correlation dk[h, j] = sum_b sum_{n >= j} dy[b, h, n] u[b, h, n - j]: per
  sequence the same correlation with u in the filter's place (``filter_grad``). The B*H input
  rows become conjugated spectra of a batch-of-one convolution of the output gradients.
- ``spectrum`` itself has no gradient and raises if its filter requires grad.
"""
from __future__ import annotations

import os
import weakref
from typing import List, Optional

import torch

from . import LONG_DEFAULT_PLANS, Plan, default_plan

PLAN_FIELDS = ("r0", "r1", "r2", "waves", "acc", "cached", "seqs", "mode", "channels")

OPS_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsffft_torch.so")
if not os.path.exists(OPS_LIB):
    raise RuntimeError(f"{OPS_LIB} is missing: build it with `make -C sffft_amd` (or __graft_entry__.build())")
torch.ops.load_library(OPS_LIB)  # defines sffft::spectrum and sffft::conv


def plan_fields(plan: Plan) -> List[int]:
    """The plan as the integer list the operators take."""
    return [int(getattr(plan, f)) for f in PLAN_FIELDS]


@torch.library.register_fake("sffft::spectrum")
def _spectrum_fake(k, plan, conj=False):
    torch._check(k.dim() == 2, lambda: "k must be [H, L]")
    torch._check(k.dtype == torch.float32, lambda: "k must be float32")
    return k.new_empty((k.shape[0], 2 * k.shape[1]), dtype=torch.complex64)


@torch.library.register_fake("sffft::conv")
def _conv_fake(u, kf, plan):
    torch._check(u.dim() == 3, lambda: "u must be [B, H, L]")
    torch._check(u.dtype in (torch.float32, torch.bfloat16), lambda: "u must be float32 or bfloat16")
    torch._check(kf.dim() == 2 and kf.shape[0] == u.shape[1] and kf.shape[1] == 2 * u.shape[2],
                 lambda: "kf must be [H, 2L]")
    return torch.empty_like(u)


def filter_grad(u: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    """dk[h, j] = sum_b sum_{n >= j} dy[b, h, n] u[b, h, n - j] for u, dy [B, H, L] (fp32 [H, L]).

    Computed on the GPU kernels per sequence as the convolution of dy with the conjugate
    spectrum of u (the correlation of the two; the conjugation is folded into the spectrum's
    gather), summed over b: the B*H rows of u are the filters (fp32 spectra) of a
    batch-of-one convolution. Multi-pass lengths (L > 16384) take
    pairs of sequences only, so there each row of dy is paired with a zero row (a batch of two
    whose second row is discarded).
    """
    B, H, L = u.shape
    pairs_only = L in LONG_DEFAULT_PLANS
    plan = default_plan(L, "fp32", 2 if pairs_only else 1)  # one sequence per transform: batch of one
    fields = plan_fields(plan)
    kf = torch.ops.sffft.spectrum(u.detach().float().reshape(B * H, L).contiguous(), fields, True)
    w = dy.float().reshape(1, B * H, L)
    if pairs_only:
        w = torch.cat([w, torch.zeros_like(w)])
    r = torch.ops.sffft.conv(w.contiguous(), kf, fields)[:1]
    return r.reshape(B, H, L).sum(0)


class _LongConvFn(torch.autograd.Function):
    """y = conv(u, kf) with gradients for u and for the filter k that kf was made from."""

    @staticmethod
    def forward(ctx, u, k, kf, fields):
        ctx.save_for_backward(u, kf)
        ctx.fields = list(fields)
        return torch.ops.sffft.conv(u, kf, fields)

    @staticmethod
    def backward(ctx, dy):
        u, kf = ctx.saved_tensors
        du = dk = None
        if ctx.needs_input_grad[0]:
            du = torch.ops.sffft.conv(dy.to(u.dtype).contiguous(), torch.conj_physical(kf), ctx.fields)
        if ctx.needs_input_grad[1]:
            dk = filter_grad(u, dy)
        return du, dk, None, None


def _drop_cached(owner_ref, key) -> None:
    owner = owner_ref()
    if owner is not None:
        owner._cache.pop(key, None)


class LongConv:
    """Causal long convolution y = causal_conv(u, k) with the filter spectrum cached.

    The spectrum of a filter tensor is kept while the tensor lives and is recomputed when it is
    modified in place (its version counter moves, as an optimizer step does) or when L or the
    plan changes. With no plan given, the tuned plan for (L, dtype, B) is used. Differentiable in
    u and, when it requires grad, in k (``filter_grad``).
    """

    def __init__(self, plan: Optional[Plan] = None):
        self._plans: dict = {}  # (L, io, B) -> (plan, its fields)
        self.plan = plan
        # id(filter) -> (weak reference to it, (version, shape, plan), spectrum); an entry is
        # dropped when its filter is freed (tensors compare elementwise, so they cannot key a
        # WeakKeyDictionary)
        self._cache: dict = {}
        self.spectra_computed = 0

    @property
    def plan(self) -> Optional[Plan]:
        return self._plan

    @plan.setter
    def plan(self, plan: Optional[Plan]) -> None:
        self._plan = plan
        self._plans.clear()

    def plan_for(self, u: torch.Tensor) -> Plan:
        return self._plan_and_fields(u)[0]

    def _plan_and_fields(self, u: torch.Tensor):
        io = "bf16" if u.dtype == torch.bfloat16 else "fp32"
        key = (u.shape[-1], io, u.shape[0])
        hit = self._plans.get(key)
        if hit is None:
            plan = self.plan if self.plan is not None else default_plan(key[0], io, key[2])
            hit = self._plans[key] = (plan, plan_fields(plan))
        return hit

    def spectrum(self, k: torch.Tensor, plan: Plan) -> torch.Tensor:
        fields = plan_fields(plan)
        key = (k._version, tuple(k.shape), tuple(fields))
        hit = self._cache.get(id(k))
        same = hit is not None and hit[0]() is k
        if same and hit[1] == key:
            return hit[2]
        kf = torch.ops.sffft.spectrum(k.detach(), fields)
        if not same:
            # the finalizer holds the cache only through a weak reference to this object, so
            # a long-lived filter does not keep a dropped LongConv's spectra alive
            weakref.finalize(k, _drop_cached, weakref.ref(self), id(k))
        self._cache[id(k)] = (weakref.ref(k), key, kf)
        self.spectra_computed += 1
        return kf

    def __call__(self, u: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
        plan, fields = self._plan_and_fields(u)
        kf = self.spectrum(k, plan)
        if k.requires_grad and torch.is_grad_enabled():
            return _LongConvFn.apply(u, k, kf, fields)
        return torch.ops.sffft.conv(u, kf, fields)
