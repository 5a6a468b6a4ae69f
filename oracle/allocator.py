"""The BatchRunner page allocator restated in Python -- TEST INFRASTRUCTURE ONLY.

Follows CudaEngine in the reference (src/cuda/cuda_runner.cu):
  free list built as num_pages-1 .. 0 so page 0 is popped first   :197
  page table zero-filled, one row of max_pages per slot           :199-204
  open_sequence: lowest closed slot, opened empty; -1 if none     :240-247
  close_sequence: pages pushed back in owned order, slot reset    :248-252
  slot(): "invalid or closed sequence id"                          :290-294
  ensure_pages: length check, then pop pages until covered        :300-313
  pages_for: ceil(tokens / 16)                                     :583
Errors are raised as AllocError(kind) with kind in {"seq", "range", "full"}.
"""
from __future__ import annotations

PAGE_SIZE = 16


class AllocError(Exception):
    def __init__(self, kind: str, msg: str):
        super().__init__(msg)
        self.kind = kind


def pages_for(tokens: int) -> int:
    return (tokens + PAGE_SIZE - 1) // PAGE_SIZE if tokens > 0 else 0


class RefAllocator:
    def __init__(self, num_pages: int, max_batch: int, max_seq_len: int):
        self.num_pages = num_pages
        self.max_batch = max_batch
        self.max_seq_len = max_seq_len
        self.max_pages = pages_for(max_seq_len)
        self.free = list(range(num_pages - 1, -1, -1))
        self.tables = [0] * (max_batch * self.max_pages)
        self.open = [False] * max_batch
        self.pages = [[] for _ in range(max_batch)]
        self.dirty = True

    def _slot(self, seq: int) -> None:
        if seq < 0 or seq >= self.max_batch or not self.open[seq]:
            raise AllocError("seq", f"invalid or closed sequence id {seq}")

    def open_sequence(self) -> int:
        for s in range(self.max_batch):
            if not self.open[s]:
                self.open[s] = True
                self.pages[s] = []
                return s
        return -1

    def close_sequence(self, seq: int) -> None:
        self._slot(seq)
        self.free.extend(self.pages[seq])
        self.open[seq] = False
        self.pages[seq] = []

    def ensure(self, seq: int, length: int) -> None:
        self._slot(seq)
        if length > self.max_seq_len:
            raise AllocError("range", "sequence longer than the maximum")
        while len(self.pages[seq]) * PAGE_SIZE < length:
            if not self.free:
                raise AllocError("full", "KV cache full: no free pages")
            page = self.free.pop()
            self.tables[seq * self.max_pages + len(self.pages[seq])] = page
            self.pages[seq].append(page)
            self.dirty = True

    @property
    def free_pages(self) -> int:
        return len(self.free)
