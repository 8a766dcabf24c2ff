"""Device descriptor (reference device.py:14-26): 'cpu', 'cuda', 'cuda:N'."""
from __future__ import annotations


class device:
    __slots__ = ("_type", "_index")

    def __init__(self, spec="cpu", index: int | None = None):
        if isinstance(spec, device):
            self._type, self._index = spec._type, spec._index
            return
        s = str(spec)
        if ":" in s:
            t, i = s.split(":", 1)
            self._type, self._index = t, int(i)
        else:
            self._type, self._index = s, index
        if self._type not in ("cpu", "cuda"):
            raise ValueError("unknown device type %r" % self._type)

    @property
    def type(self) -> str:
        return self._type

    @property
    def index(self) -> int | None:
        return self._index

    @property
    def is_cuda(self) -> bool:
        return self._type == "cuda"

    def ordinal(self) -> int:
        return self._index if self._index is not None else 0

    def __eq__(self, other) -> bool:
        o = device(other)
        return self._type == o._type and (self._type == "cpu" or self.ordinal() == o.ordinal())

    def __hash__(self) -> int:
        return hash((self._type, self.ordinal() if self._type == "cuda" else None))

    def __repr__(self) -> str:
        return "device(%r)" % str(self)

    def __str__(self) -> str:
        return self._type if self._index is None else "%s:%d" % (self._type, self._index)
