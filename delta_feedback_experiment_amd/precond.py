"""Preconditioner scan host side (kernels pending in this build)."""

from __future__ import annotations


def precond_forward(*args, **kwargs):
    raise NotImplementedError("the preconditioner scan is not built yet")


def precond_backward(*args, **kwargs):
    raise NotImplementedError("the preconditioner scan is not built yet")
