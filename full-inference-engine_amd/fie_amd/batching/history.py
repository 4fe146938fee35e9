"""Penalty histories kept on the device across steps.

The reference rebuilds every penalised row's seen-token table on the host at every
step (engine/batching/sampler.py:134-155): O(rows x context) Python work and a
fresh upload, although a decoding request's context only grows by one token per
step (engine/batching/continuous_batching.py:1920-1925 passes prompt + output).
``DeviceHistory`` keeps each request's context in one device array instead and
uploads only what was appended since the request's last step; the kernels read
each row's [start, end) range of that array (``fie_sampler_args.hist_ends``).

Contract: a request id's context only grows between steps (prompt + output, as
the engine builds it), or the id is forgotten (``forget``) before its context
changes otherwise.  Cheap probes catch the usual violations and store such a
context afresh: a context shorter than the stored one, a change among the last
kTail stored tokens (a rollback), or at the first token or at three positions
fixed when the context was stored (a reused id).  A change elsewhere in a long
context is not detected in O(1) per row.
"""

from __future__ import annotations

import operator

import numpy as np
import torch


kTail = 8   # stored tokens compared at every step, counted from the end


class _Slot:
    __slots__ = ("start", "cap", "length", "tail", "probe_get", "probe_vals", "vocab", "bigs",
                 "zero", "late")

    def __init__(self, start: int, cap: int, vocab: int):
        self.start, self.cap, self.length, self.vocab = start, cap, 0, vocab
        self.tail: list[int] = []                  # the last kTail stored ids
        self.probe_get = None                      # itemgetter of the positions fixed at storing
        self.probe_vals: tuple = ()                # the ids stored there
        self.bigs: set[int] = set()   # distinct ids >= vocab seen
        self.zero: int | None = None  # position of the first token 0
        self.late = False             # an id >= vocab first occurs after the first 0

    def extended_by(self, ctx: list[int], n: int) -> bool:
        """Whether ctx (length n) holds the stored context as its prefix, by the
        probes of the module contract."""
        ln = self.length
        if n < ln:
            return False
        if ln == 0:
            return True
        if ctx[ln - kTail if ln > kTail else 0:ln] != self.tail:
            return False
        return self.probe_get(ctx) == self.probe_vals

    def stored(self, ctx: list[int], n: int) -> None:
        """Record that ctx[:n] is now the stored context."""
        if self.length == 0 and n:
            at = sorted({0, n // 4, n // 2, (3 * n) // 4})
            # two positions at least, so the getter always returns a tuple
            at = at if len(at) > 1 else at * 2
            self.probe_get = operator.itemgetter(*at)
            self.probe_vals = self.probe_get(ctx)
        self.length = n
        self.tail = ctx[n - kTail if n > kTail else 0:n]


class DeviceHistory:
    """Per-request contexts in one int32 device array (a bump arena).

    A step first decides, for every row, whether its request needs fresh space (a
    new context, or one that outgrew its slot), then makes room for all of it at
    once (growing or compacting the array, which moves slots), and only then hands
    out space and records the rows' ranges and write positions: nothing recorded in
    a step can be moved by a later row of the same step."""

    # set once any stored context holds an id >= vocab: only then do rows need the
    # out-of-vocabulary scan of update()
    _with_bigs = False

    def __init__(self, device: torch.device, capacity: int = 1 << 20):
        self.device = device
        self.ids = torch.empty(capacity, dtype=torch.int32, device=device)
        self.top = 0
        self.live = 0
        self.slots: dict[object, _Slot] = {}

    # ------------------------------------------------------------------ storage
    def _make_room(self, n: int) -> None:
        """Ensure n free ints past `top`, growing (or compacting) the array; live
        slots may move (their `start` is updated)."""
        if self.top + n <= self.ids.numel():
            return
        size = max(2 * self.ids.numel(), 2 * (self.live + n))
        fresh = torch.empty(size, dtype=torch.int32, device=self.device)
        if self.top - self.live > self.live:
            # mostly dead space: move the live slots down
            at = 0
            for slot in self.slots.values():
                fresh[at:at + slot.length].copy_(self.ids[slot.start:slot.start + slot.length])
                slot.start = at
                at += slot.cap
            self.top = at
        else:
            fresh[:self.top].copy_(self.ids[:self.top])
        self.ids = fresh

    def _bump(self, n: int) -> int:
        """Start of n free ints; _make_room has reserved them (nothing moves)."""
        at = self.top
        self.top += n
        if self.top > self.ids.numel():
            raise AssertionError("DeviceHistory: space handed out beyond the room made for the step")
        return at

    @staticmethod
    def _new_cap(n: int) -> int:
        return max(256, 2 * n)

    @staticmethod
    def _grow_cap(slot: _Slot, n: int) -> int:
        return max(2 * slot.cap, 2 * n)

    def _new_slot(self, rid: object, cap: int, vocab: int) -> _Slot:
        old = self.slots.pop(rid, None)
        if old is not None:
            self.live -= old.cap
        slot = _Slot(self._bump(cap), cap, vocab)
        self.slots[rid] = slot
        self.live += cap
        return slot

    def _grow(self, slot: _Slot, cap: int) -> None:
        start = self._bump(cap)
        self.ids[start:start + slot.length].copy_(self.ids[slot.start:slot.start + slot.length])
        self.live += cap - slot.cap
        slot.start, slot.cap = start, cap

    def forget(self, request_ids: list[object]) -> None:
        for rid in request_ids:
            slot = self.slots.pop(rid, None)
            if slot is not None:
                self.live -= slot.cap

    # ------------------------------------------------------------------ one step
    @staticmethod
    def _note(slot: _Slot, new: np.ndarray, vocab: int, base: int | None = None) -> None:
        """Token-0 bookkeeping of sampler.py:148,156-157 over ids appended at
        position `base` (the slot's length before them, by default)."""
        if not new.size:
            return
        base = slot.length if base is None else base
        zeros = np.nonzero(new == 0)[0]
        big = np.nonzero(new >= vocab)[0]
        if slot.zero is None and zeros.size:
            slot.zero = base + int(zeros[0])
        for p in big.tolist():
            t = int(new[p])
            if t not in slot.bigs:
                slot.bigs.add(t)
                DeviceHistory._with_bigs = True
                if slot.zero is not None and base + p > slot.zero:
                    slot.late = True

    def update(self, contexts: list[list[int]], include: np.ndarray, request_ids: list[object],
               vocab: int):
        """Bring the penalised rows' stored contexts up to date.  Returns (starts,
        ends, hist_invalid or None, longest, write_dst, write_src): the rows'
        ranges in ``ids`` and the appended tokens still to be written there.

        One pass decides each row's action and the room the step needs; after the
        room is made, a second pass hands out space and gathers the appended ids
        into one list; the range check and the token-0 scan then run once over all
        of them, and the slots advance only after the check passes."""
        rows = len(contexts)
        sel = np.flatnonzero(include).tolist()
        picked = [request_ids[r] for r in sel]
        if len(set(picked)) != len(picked):
            # one request twice in a batch: rows see each other's appends in order
            return self._update_rowwise(contexts, include, request_ids, vocab)
        fast = self._update_fast(contexts, sel, picked, rows, vocab)
        if fast is not None:
            return fast
        get = self.slots.get
        # pass 1: each row's action (0 keep, 1 new slot, 2 grow) and the room needed
        acts = []
        need = 0
        for r, rid in zip(sel, picked):
            ctx = contexts[r]
            n = len(ctx)
            slot = get(rid)
            if slot is None or slot.vocab != vocab or not slot.extended_by(ctx, n):
                cap = self._new_cap(n)
                acts.append((1, cap))
                need += cap
            elif n > slot.cap:
                cap = self._grow_cap(slot, n)
                acts.append((2, cap))
                need += cap
            else:
                acts.append((0, 0))
        self._make_room(need)
        # pass 2: space handed out (nothing moves now), appended ids gathered
        starts_l = [0] * rows
        ends_l = [0] * rows
        longest = 0
        flat: list[int] = []
        moved = []            # (slot, old length, new length, context) of rows that grew
        counts, bases = [], []
        extend, c_append, b_append, m_append = flat.extend, counts.append, bases.append, moved.append
        for (r, rid), (act, cap) in zip(zip(sel, picked), acts):
            ctx = contexts[r]
            n = len(ctx)
            if act == 1:
                slot = self._new_slot(rid, cap, vocab)
            else:
                slot = self.slots[rid]
                if act == 2:
                    self._grow(slot, cap)
            ln = slot.length
            st = slot.start
            if n > ln:
                extend(ctx[ln:])
                c_append(n - ln)
                b_append(st + ln)
                m_append((slot, ln, n, ctx))
            starts_l[r] = st
            ends_l[r] = st + n
            if n > longest:
                longest = n
        return self._finish_update(contexts, sel, picked, rows, vocab, starts_l, ends_l, longest,
                                   flat, counts, bases, moved)

    def _update_fast(self, contexts, sel, picked, rows, vocab):
        """update() when every row's request has a slot holding a prefix of its
        context with room for the rest (the steady state of decoding): one pass and
        no slot moves; None when some row needs a new or larger slot."""
        get = self.slots.get
        starts_l = [0] * rows
        ends_l = [0] * rows
        longest = 0
        flat: list[int] = []
        moved = []
        counts, bases = [], []
        extend, c_append, b_append, m_append = flat.extend, counts.append, bases.append, moved.append
        for r, rid in zip(sel, picked):
            ctx = contexts[r]
            n = len(ctx)
            slot = get(rid)
            if slot is None or slot.vocab != vocab or n > slot.cap:
                return None
            ln = slot.length
            if ln:
                if n < ln or ctx[ln - kTail if ln > kTail else 0:ln] != slot.tail \
                        or slot.probe_get(ctx) != slot.probe_vals:
                    return None
            st = slot.start
            if n > ln:
                extend(ctx[ln:])
                c_append(n - ln)
                b_append(st + ln)
                m_append((slot, ln, n, ctx))
            starts_l[r] = st
            ends_l[r] = st + n
            if n > longest:
                longest = n
        return self._finish_update(contexts, sel, picked, rows, vocab, starts_l, ends_l, longest,
                                   flat, counts, bases, moved)

    def _finish_update(self, contexts, sel, picked, rows, vocab, starts_l, ends_l, longest,
                       flat, counts, bases, moved):
        """The common tail of update(): range check and token-0 bookkeeping over all
        appended ids at once, then the slots advance."""
        starts = np.array(starts_l, dtype=np.int64)
        ends = np.array(ends_l, dtype=np.int64)
        if flat:
            new = np.asarray(flat, dtype=np.int64)
            if int(new.min()) < 0 or int(new.max()) >= 2**31:
                raise ValueError("penalty context token ids must be in [0, 2**31)")
            cnt = np.asarray(counts, dtype=np.int64)
            first = np.cumsum(cnt) - cnt                      # each row's offset in `new`
            dst = np.repeat(np.asarray(bases, dtype=np.int64) - first, cnt) + np.arange(new.size)
            src = new.astype(np.int32)
            odd = (new == 0) | (new >= vocab)
            if odd.any():
                seg = np.repeat(np.arange(cnt.size), cnt)
                for i in np.unique(seg[odd]).tolist():
                    slot, old, _, _ = moved[i]
                    self._note(slot, new[first[i]:first[i] + cnt[i]], vocab, base=old)
            for slot, _, n, ctx in moved:
                slot.stored(ctx, n)
        else:
            dst = np.zeros(0, np.int64)
            src = np.zeros(0, np.int32)
        invalid = None
        if self._with_bigs:
            slots = self.slots
            for r, rid in zip(sel, picked):
                slot = slots[rid]
                if slot.bigs:
                    if invalid is None:
                        invalid = np.zeros(rows, dtype=np.int32)
                    invalid[r] = len(slot.bigs) | ((1 << 30) if slot.late else 0)
        return starts, ends, invalid, longest, dst, src

    def _update_rowwise(self, contexts: list[list[int]], include: np.ndarray,
                        request_ids: list[object], vocab: int):
        """update() one row after another (a request that appears twice).  The room
        is made first for the allocations a dry run of the rows predicts, so no
        slot moves while rows are recorded, and a slot one row replaces keeps its
        memory until the step ends."""
        rows = len(contexts)
        # dry run: per request, (cap, length, vocab, context) as the rows leave it
        sim: dict[object, tuple] = {}
        need = 0
        for r in range(rows):
            if not include[r]:
                continue
            ctx = contexts[r]
            n = len(ctx)
            rid = request_ids[r]
            if rid in sim:
                cap, ln, voc, prev = sim[rid]
                ext = voc == vocab and n >= ln and ctx[:ln] == prev[:ln]
            else:
                slot = self.slots.get(rid)
                cap = slot.cap if slot is not None else 0
                ext = slot is not None and slot.vocab == vocab and slot.extended_by(ctx, n)
            if not ext:
                cap = self._new_cap(n)
                need += cap
            elif n > cap:
                cap = max(2 * cap, 2 * n)
                need += cap
            sim[rid] = (cap, n, vocab, ctx)
        self._make_room(need)
        starts = np.zeros(rows, dtype=np.int64)
        ends = np.zeros(rows, dtype=np.int64)
        invalid = np.zeros(rows, dtype=np.int32)
        longest = 0
        dst_parts, src_parts = [], []
        for r in range(rows):
            if not include[r]:
                continue
            ctx = contexts[r]
            n = len(ctx)
            rid = request_ids[r]
            slot = self.slots.get(rid)
            if slot is None or slot.vocab != vocab or not slot.extended_by(ctx, n):
                slot = self._new_slot(rid, self._new_cap(n), vocab)
            elif n > slot.cap:
                self._grow(slot, self._grow_cap(slot, n))
            if n > slot.length:
                new = np.asarray(ctx[slot.length:], dtype=np.int64)
                if new.min() < 0 or new.max() >= 2**31:
                    raise ValueError("penalty context token ids must be in [0, 2**31)")
                self._note(slot, new, vocab)
                dst_parts.append(np.arange(slot.start + slot.length, slot.start + n, dtype=np.int64))
                src_parts.append(new.astype(np.int32))
                slot.stored(ctx, n)
            starts[r] = slot.start
            ends[r] = slot.start + n
            if slot.bigs:
                invalid[r] = len(slot.bigs) | ((1 << 30) if slot.late else 0)
            longest = max(longest, n)
        dst = np.concatenate(dst_parts) if dst_parts else np.zeros(0, np.int64)
        src = np.concatenate(src_parts) if src_parts else np.zeros(0, np.int32)
        return starts, ends, (invalid if invalid.any() else None), longest, dst, src
