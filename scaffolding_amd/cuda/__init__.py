"""Device runtime helpers (reference cuda/__init__.py:45-303): availability,
device selection, synchronisation, events, allocator cache."""
from __future__ import annotations

from .. import _cuda_ops as _cuops


def manual_seed(seed: int) -> None:
    """Seeds the device random stream that dropout draws from (reference
    cuda/__init__.py:366-368, a no-op there)."""
    _cuops.manual_seed(int(seed))


def manual_seed_all(seed: int) -> None:
    """One random stream serves every device (reference
    cuda/__init__.py:371-373)."""
    _cuops.manual_seed(int(seed))


def is_available() -> bool:
    return _cuops.get_device_count() > 0


def device_count() -> int:
    return _cuops.get_device_count()


def set_device(device: int) -> None:
    _cuops.set_device(int(device))


def current_device() -> int:
    return _cuops.get_current_device()


def synchronize(device=None) -> None:
    """reference cuda/__init__.py:135-144."""
    _cuops.device_synchronize()


def get_device_name(device: int = 0) -> str:
    return _cuops.get_device_name(device)


def get_device_properties(device: int = 0) -> dict:
    return _cuops.get_device_properties(device)


def empty_cache() -> None:
    _cuops.empty_cache(-1)


def memory_stats() -> dict:
    """Pooled and live bytes of the native caching allocator (the
    reference's stats are never incremented, cuda/__init__.py:151-213)."""
    pooled, live = _cuops.cache_stats(-1)
    return {"pooled_bytes": pooled, "allocated_bytes": live}


def memory_allocated(device=None) -> int:
    return _cuops.cache_stats(-1 if device is None else int(device))[1]


class Stream:
    """reference cuda/__init__.py:252-280."""

    def __init__(self, device: int = 0):
        self._s = _cuops.CudaStream(device)

    def synchronize(self) -> None:
        self._s.synchronize()

    def wait_event(self, event: "Event") -> None:
        self._s.wait_event(event._e)

    @property
    def cuda_stream(self) -> int:
        return self._s.cuda_stream


class Event:
    """reference cuda/__init__.py:281-303; elapsed_time in milliseconds."""

    def __init__(self, enable_timing: bool = True):
        self._e = _cuops.CudaEvent(enable_timing)

    def record(self, stream: Stream | None = None) -> None:
        self._e.record(None if stream is None else stream._s)

    def synchronize(self) -> None:
        self._e.synchronize()

    def elapsed_time(self, end: "Event") -> float:
        return self._e.elapsed_time(end._e)
