"""Candidate streaming: gated products whose packed candidates live in host
memory, copied into a ring of device slots on a copy stream ahead of use.

The reference keeps candidates on the host and copies each one host -> device
in every forward and again in every backward (``layers.py:348, 362``; its
lazy path the same for the packed bytes unless ``--qbytes_device``), in
stream order, so each copy sits in front of the product that needs it.  It
dropped a side stream after aperture violations from unfenced side-stream
use (``layers.py:524-529``).

Here, when a model's candidates do not stay resident in HBM (a model whose K
candidates exceed the GPU's memory), a :class:`CandidateStreamer` keeps each
gated product's packed bytes in pinned host memory and overlaps their copies
with the products before them:

* A *product* is what one launch reads: a gated Linear, or the members of a
  stacked projection (q/k/v, gate/up).  Products are numbered in forward
  order; product i always uses device slot i mod R (R slots of the largest
  product's bytes), so the views its autograd Function keeps for the backward
  point at the same memory then.
* A fence runs before each product: in the forward, in the module's forward;
  in the backward, as the backward of an identity Function applied to the
  product's output, which autograd runs just before the product's own
  backward.  The fence records an event on the compute stream (everything
  enqueued before this product), makes the compute stream wait for this
  product's copy, and issues the copies of the next D products (forward:
  i + 1 .. i + D; backward: i - 1 .. i - D) on the copy stream, each behind
  the fence's event.  With D < R the previous user of each of those slots is
  a product the fence's event already covers.
* A slot still holding a product's bytes is reused without a copy (the last
  products of the forward are the first of the backward, and product 0 opens
  the next step).
* ``overlap=False`` copies on the compute stream in stream order, the
  reference's pattern, for comparison: the same kernels on the same bytes,
  so both modes give bit-identical results.

Every stream is created at the default priority.
"""

from __future__ import annotations

import torch
from torch.autograd import Function

_ALIGN = 256  # bytes: every candidate view starts 256-byte aligned


class _BackwardFence(Function):
    """Identity on a product's output; its backward (which autograd runs just
    before the product's backward) runs the streamer's backward fence."""

    @staticmethod
    def forward(ctx, y, streamer, index):
        ctx.streamer = streamer
        ctx.index = index
        return y.view_as(y)

    @staticmethod
    def backward(ctx, g):
        ctx.streamer.fence(ctx.index, backward=True)
        return g, None, None


class CandidateStreamer:
    """Streams the packed candidates of `products` (lists of gated Linears,
    in forward order) from pinned host memory through `slots` device slots,
    `depth` products ahead, on a copy stream of default priority."""

    def __init__(self, products: list[list], device, slots: int = 4, depth: int = 2, overlap: bool = True,
                 timeline: bool = False):
        if not products:
            raise ValueError("no products to stream")
        if not 1 <= depth < slots:
            raise ValueError(f"need 1 <= depth < slots (got depth={depth}, slots={slots})")
        self.device = torch.device(device)
        self.products = [list(p) for p in products]
        self.slots_n = int(slots)
        self.depth = int(depth)
        self.overlap = bool(overlap)
        self.index: dict[int, int] = {}
        self.layout: list[list[list[tuple[int, int]]]] = []  # product -> member -> [(offset, bytes)] per candidate
        sizes = []
        for i, mods in enumerate(self.products):
            off, lay = 0, []
            for m in mods:
                if id(m) in self.index:
                    raise ValueError(f"{m._tensor_name} appears in two products")
                self.index[id(m)] = i
                spans = []
                for qb in m._qbytes():
                    spans.append((off, qb.numel()))
                    off += (qb.numel() + _ALIGN - 1) // _ALIGN * _ALIGN
                lay.append(spans)
            self.layout.append(lay)
            sizes.append(off)
        self.slot_bytes = max(sizes)
        self.product_bytes = sizes
        # host copies (pinned) of every candidate; the modules stop holding device bytes
        self.host: list[list[list[torch.Tensor]]] = []
        for mods in self.products:
            hp = []
            for m in mods:
                hq = []
                for k, qb in enumerate(m._qbytes()):
                    h = torch.empty(qb.numel(), dtype=torch.uint8, pin_memory=True)
                    h.copy_(qb.reshape(-1))
                    hq.append(h)
                    setattr(m, f"_qweight_{k}", h)
                m._streamer = self
                hp.append(hq)
            self.host.append(hp)
        self.slot_mem = [torch.empty(self.slot_bytes, dtype=torch.uint8, device=self.device)
                         for _ in range(self.slots_n)]
        self.resident = [-1] * self.slots_n  # product whose bytes each slot holds
        self.ready: list[torch.cuda.Event | None] = [None] * len(self.products)
        self.copy_stream = torch.cuda.Stream(device=self.device) if self.overlap else None
        self.bytes_copied = 0
        # timeline=True: timing events around every copy and after every fence
        # (see timeline_ms); off by default, as each costs two event records
        self.timeline: list | None = [] if timeline else None

    # -- views handed to the autograd Functions ------------------------------
    def views(self, module) -> list[torch.Tensor]:
        i = self.index[id(module)]
        j = next(k for k, m in enumerate(self.products[i]) if m is module)
        mem = self.slot_mem[i % self.slots_n]
        return [mem[off:off + n] for off, n in self.layout[i][j]]

    def fenced(self, y: torch.Tensor, module) -> torch.Tensor:
        """The product's output, through the backward fence."""
        return _BackwardFence.apply(y, self, self.index[id(module)])

    # -- fences ----------------------------------------------------------------
    def _copy(self, i: int, stream) -> None:
        s = i % self.slots_n
        mem = self.slot_mem[s]
        with torch.cuda.stream(stream):
            if self.timeline is not None:
                start = torch.cuda.Event(enable_timing=True)
                start.record(stream)
            for hq, spans in zip(self.host[i], self.layout[i]):
                for h, (off, n) in zip(hq, spans):
                    mem[off:off + n].copy_(h, non_blocking=True)
            ev = torch.cuda.Event(enable_timing=self.timeline is not None)
            ev.record(stream)
        if self.timeline is not None:
            self.timeline.append(("copy", i, start, ev))
        self.ready[i] = ev
        self.resident[s] = i
        self.bytes_copied += self.product_bytes[i]

    def fence(self, i: int, backward: bool) -> None:
        self._fence(i, backward)
        if self.timeline is not None:
            passed = torch.cuda.Event(enable_timing=True)
            passed.record(torch.cuda.current_stream(self.device))
            self.timeline.append(("backward" if backward else "forward", i, passed, None))

    def _fence(self, i: int, backward: bool) -> None:
        compute = torch.cuda.current_stream(self.device)
        s = i % self.slots_n
        if not self.overlap:
            if self.resident[s] != i:
                self._copy(i, compute)
            return
        if self.resident[s] != i:  # not prefetched (the first product, or a cold start)
            before = torch.cuda.Event()
            before.record(compute)
            self.copy_stream.wait_event(before)
            self._copy(i, self.copy_stream)
        compute.wait_event(self.ready[i])
        ahead = [i - d for d in range(1, self.depth + 1)] if backward else [i + d for d in range(1, self.depth + 1)]
        ahead = [j for j in ahead if 0 <= j < len(self.products) and self.resident[j % self.slots_n] != j]
        if ahead:
            before = torch.cuda.Event()
            before.record(compute)
            self.copy_stream.wait_event(before)
            for j in ahead:
                self._copy(j, self.copy_stream)

    def timeline_ms(self, origin: torch.cuda.Event) -> list[tuple]:
        """The recorded copies and fences (timeline=True) as milliseconds after
        `origin`, a timing event recorded on the compute stream before them:
        ("copy", product, start, end) and ("forward" | "backward", product,
        time the compute stream passed the fence, None).  Call once the device
        has finished the recorded work; clears the record."""
        if self.timeline is None:
            raise ValueError("the streamer was built without timeline=True")
        out = [(kind, i, origin.elapsed_time(a), origin.elapsed_time(b) if b is not None else None)
               for kind, i, a, b in self.timeline]
        self.timeline.clear()
        return out

    def forward_fence(self, module) -> None:
        self.fence(self.index[id(module)], backward=False)

    def synchronize(self) -> None:
        """The compute stream waits for every queued copy."""
        if self.copy_stream is not None:
            torch.cuda.current_stream(self.device).wait_stream(self.copy_stream)

    def release(self) -> None:
        """Give the modules resident device copies of their candidates back."""
        self.synchronize()
        for mods, hp in zip(self.products, self.host):
            for m, hq in zip(mods, hp):
                for k, h in enumerate(hq):
                    setattr(m, f"_qweight_{k}", h.to(self.device))
                m._streamer = None
        self.slot_mem = []
