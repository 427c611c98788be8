"""Exceptions raised by the package (the reference's classes, packed_encoders/errors.py:11-20).

A refusal is always one of these, never a quiet downgrade to another kernel.
"""

from __future__ import annotations


class PackedEncodersError(Exception):
    """Base class for every error this package raises."""


class UnsupportedTargetError(PackedEncodersError):
    """`pack()` could not locate a supported encoder, or a piece rejects its inputs."""


class ValidationError(PackedEncodersError):
    """A validation gate failed — the fused path was refused."""
