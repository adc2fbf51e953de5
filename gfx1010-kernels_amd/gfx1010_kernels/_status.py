"""Backend status record returned by the diagnostic API.

Same fields and semantics as the reference's ``BackendStatus``
(gfx1010_kernels/attention.py:14-19).
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class BackendStatus:
    available: bool
    device: str | None
    architecture: str | None
    reason: str
