"""Dispatch ledger: which native arm each op call took.

Restates python/minisgl/_hip_engage.py:49-71 of the reference: ``engaged(name)`` tallies every
host-side dispatch; ``counts()`` snapshots the tally and ``counts_delta(before)`` returns the arms
that moved. Under HIP-graph replay the counts do not move (replays never re-enter Python).
"""
from __future__ import annotations

import logging
import os

_log = logging.getLogger("w4a8.hip-engage")
_seen: set[str] = set()
_ON = os.environ.get("MINISGL_HIP_ENGAGE_LOG", "1") != "0"

COUNTS: dict[str, int] = {}


def engaged(name: str) -> None:
    COUNTS[name] = COUNTS.get(name, 0) + 1
    if _ON and name not in _seen:
        _seen.add(name)
        _log.info("[hip-engage] %s", name)


def counts() -> dict[str, int]:
    return dict(COUNTS)


def counts_delta(before: dict[str, int]) -> dict[str, int]:
    now = counts()
    keys = set(now) | set(before)
    return {k: now.get(k, 0) - before.get(k, 0) for k in sorted(keys) if now.get(k, 0) != before.get(k, 0)}
