"""Prepared-page cache for ``hip_mi355x``: reference ``dotcache/page_cache.py:23-227``.

Keeps the device-resident copy of each host page it has prepared, keyed by
the host page's identity (reference ``page_cache.py:155``, ``:198``), so a
decode loop that passes the same ``EncodedPage`` objects every step uploads
them once.  A byte budget (``max_resident_bytes``) bounds what the cache
holds; past it, entries are dropped in the order the policy gives:

``fifo``                oldest inserted first;
``lru``                 least recently returned first (a hit moves an entry
                        to the back, reference ``page_cache.py:62-64``);
``pinned_recent_fifo``  oldest inserted first, skipping the
                        ``pinned_recent_pages`` newest entries while any
                        older one is left; when every entry is pinned the
                        oldest goes (reference ``page_cache.py:53-104``).

An entry's size is the page's blob in its device pool (``resident_nbytes``;
the host-to-device byte count when that is zero, reference
``page_cache.py:47-51``).  Dropping an entry drops the cache's reference to
the prepared page; the blob returns to its pool when the last reference
goes, so a page the caller still holds stays valid and a budget-bounded
cache keeps its pools bounded.

Differences from the reference, both deliberate: a page listed twice among
the misses of one ``prepare_pages`` call is uploaded once (the reference
uploads it twice and counts its bytes twice), and backend ``"auto"`` never
falls back to the CPU -- without a GPU the preparer raises RuntimeError,
as every entry point of this package does.
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Any, Callable, Literal, Sequence

from .backends.hip_mi355x import DEVICE_TYPE, PreparedPageHIP, prepare_pages_hip
from .tracing import ExecutionTrace
from .types import EncodedPage

CachePolicy = Literal["fifo", "lru", "pinned_recent_fifo"]
CacheBackend = Literal["auto", "hip_mi355x"]
PageLike = EncodedPage | PreparedPageHIP
_POLICIES = ("fifo", "lru", "pinned_recent_fifo")


@dataclass(slots=True)
class PreparedPageCache:
    """Reference ``PreparedPageCache`` (``page_cache.py:23-227``) for the
    ``hip_mi355x`` backend.  ``preparer`` uploads a list of host pages and
    returns their prepared pages; it defaults to ``prepare_pages_hip``."""

    max_resident_bytes: int | None = None
    policy: CachePolicy = "fifo"
    pinned_recent_pages: int = 0
    preparer: Callable[..., list[Any]] | None = None
    _entries: OrderedDict = field(default_factory=OrderedDict)  # (device, id(host page)) -> prepared page
    _owned: set = field(default_factory=set)  # id() of the prepared pages held
    _resident_bytes: int = 0

    def __post_init__(self) -> None:
        if self.policy not in _POLICIES:
            raise ValueError(f"unknown cache policy {self.policy!r}; expected one of {_POLICIES}")
        if self.max_resident_bytes is not None and int(self.max_resident_bytes) < 0:
            raise ValueError("max_resident_bytes must be non-negative")
        if int(self.pinned_recent_pages) < 0:
            raise ValueError("pinned_recent_pages must be non-negative")

    # ---- the reference's public surface --------------------------------
    @property
    def resident_bytes(self) -> int:
        return self._resident_bytes

    @property
    def size(self) -> int:
        return len(self._entries)

    def clear(self) -> None:
        self._entries.clear()
        self._owned.clear()
        self._resident_bytes = 0

    def owns_prepared_page(self, page: Any) -> bool:
        return id(page) in self._owned

    def append_page(self, page: PageLike, *, backend: CacheBackend = "auto",
                    trace: ExecutionTrace | None = None) -> PreparedPageHIP:
        return self.prepare_page(page, backend=backend, trace=trace)

    def append_pages(self, pages: Sequence[PageLike], *, backend: CacheBackend = "auto",
                     trace: ExecutionTrace | None = None) -> list[PreparedPageHIP]:
        return self.prepare_pages(pages, backend=backend, trace=trace)

    def prepare_page(self, page: PageLike, *, backend: CacheBackend = "auto",
                     trace: ExecutionTrace | None = None) -> PreparedPageHIP:
        return self.prepare_pages([page], backend=backend, trace=trace)[0]

    def prepare_pages(self, pages: Sequence[PageLike], *, backend: CacheBackend = "auto",
                      trace: ExecutionTrace | None = None) -> list[PreparedPageHIP]:
        """Prepared pages for ``pages`` in order: already-prepared pages and
        cached ones are hits; the misses go to the device in one batch and
        are inserted oldest-first, each after making room for itself."""
        if backend not in ("auto", "hip_mi355x"):
            raise ValueError(f"unknown backend {backend!r} (this cache serves hip_mi355x)")
        out: list[Any] = [None] * len(pages)
        misses: dict[int, list[int]] = {}  # id(host page) -> positions in ``pages``
        for i, page in enumerate(pages):
            if isinstance(page, PreparedPageHIP):
                out[i] = page
                self._hit(trace)
                continue
            key = (DEVICE_TYPE, id(page))
            cached = self._entries.get(key)
            if cached is not None:
                if self.policy == "lru":
                    self._entries.move_to_end(key)
                out[i] = cached
                self._hit(trace)
            elif id(page) in misses:
                misses[id(page)].append(i)
                self._hit(trace)
            else:
                misses[id(page)] = [i]
        if misses:
            sources = [pages[pos[0]] for pos in misses.values()]
            prepared = (self.preparer or prepare_pages_hip)(sources, trace=trace)
            if len(prepared) != len(sources):
                raise RuntimeError("prepared page cache failed to populate all requested pages")
            for src, pp, pos in zip(sources, prepared, misses.values()):
                nbytes = self._nbytes(pp)
                self._make_room(nbytes, trace)
                self._entries[(DEVICE_TYPE, id(src))] = pp
                self._owned.add(id(pp))
                self._resident_bytes += nbytes
                for i in pos:
                    out[i] = pp
                if trace is not None:
                    trace.record_cache_miss()
                    trace.observe_cache_resident_bytes(self._resident_bytes)
        return out

    # ---- policy ------------------------------------------------------------
    def _hit(self, trace: ExecutionTrace | None) -> None:
        if trace is not None:
            trace.record_cache_hit()
            trace.observe_cache_resident_bytes(self._resident_bytes)

    @staticmethod
    def _nbytes(page: Any) -> int:
        n = int(page.resident_nbytes)
        return n if n > 0 else int(page.host_to_device_nbytes)

    def _victim(self):
        """The key the policy drops next.  That is always the front entry:
        under ``lru`` the front is the least recently returned; under the
        FIFO policies entries keep insertion order, and the pinned entries
        are the newest ones, so the oldest entry is unpinned whenever any
        entry is, and is the all-pinned fallback otherwise."""
        return next(iter(self._entries))

    def _make_room(self, incoming: int, trace: ExecutionTrace | None) -> None:
        if self.max_resident_bytes is None:
            return
        while self._entries and self._resident_bytes + incoming > int(self.max_resident_bytes):
            key = self._victim()
            page = self._entries.pop(key)
            self._owned.discard(id(page))
            nbytes = self._nbytes(page)
            self._resident_bytes = max(0, self._resident_bytes - nbytes)
            if trace is not None:
                trace.record_cache_eviction(nbytes)
                trace.observe_cache_resident_bytes(self._resident_bytes)
