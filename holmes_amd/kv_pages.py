"""PairFold128 decode KV cache on HBM-resident pages.

The ownership surface follows llama3fhe/operators/pairfold_kv_cache.py (PairFoldTokenWrite,
PairFoldCipherPage, PairFoldLayerCache, drop_pairfold_token_to_limbs; lines 1-621): a token write
owns four ciphertexts (two key groups, two value groups) for one of a page's 128 columns; the first
token of a page becomes the page by move; every later token of the page is added into it, the four
sums committed together only after all exist, then the old tail and the token are released; full
pages are never copied.  Every failure before the commit leaves both owners unchanged.

On this backend the pages live in a KVPagePool: one HBM allocation of page slots
``[capacity][4][2][limbs][N]`` (four ciphertexts, two components).  A page's ciphertexts are views
into its slot, and the partial-page append writes the four sums into a fresh slot with one
hck_lincomb launch (eight polynomial sums), instead of four separate allocations and eight add
kernels; the old tail's slot is returned to the pool when its ciphertexts are released.  Without a
pool (or for ciphertexts of another backend) the append goes through ``crypto_context.fhe.homo_add``
exactly as the reference does.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable

import torch

from .context import Cipher, u64_clone

PAIRFOLD_LAYOUT_TAG = "pairfold128_v1"
PAIRFOLD_PAGE_SIZE = 128
PAIRFOLD_GROUP_COUNT = 2
_HANDLES = 2 * PAIRFOLD_GROUP_COUNT

__all__ = [
    "PAIRFOLD_GROUP_COUNT",
    "PAIRFOLD_LAYOUT_TAG",
    "PAIRFOLD_PAGE_SIZE",
    "KVPagePool",
    "PooledCipher",
    "PairFoldCipherPage",
    "PairFoldLayerCache",
    "PairFoldTokenWrite",
    "drop_pairfold_token_to_limbs",
]


# ---------------------------------------------------------------------------- ownership primitives
def _free(handles: Iterable[object]) -> BaseException | None:
    """Call ``release()`` once on every distinct handle (in order), whatever fails on the way;
    hand back the first exception instead of raising it."""

    done: set[int] = set()
    first: BaseException | None = None
    for h in handles:
        if id(h) in done:
            continue
        done.add(id(h))
        release = getattr(h, "release", None)
        if not callable(release):
            continue
        try:
            release()
        except BaseException as exc:  # keep releasing the rest
            first = exc if first is None else first
    return first


def _distinct(handles: Iterable[object], what: str) -> tuple:
    items = tuple(handles)
    if len(set(map(id, items))) < len(items):
        raise ValueError(f"{what}: the same ciphertext object appears twice (handles alias)")
    return items


def _groups(values: Iterable[object], what: str) -> tuple:
    items = tuple(values)
    if len(items) != PAIRFOLD_GROUP_COUNT or any(v is None for v in items):
        raise ValueError(f"{what} needs {PAIRFOLD_GROUP_COUNT} ciphertexts (no None), got {len(items)}")
    return items


class _Staged:
    """Ciphertexts produced inside one transaction.  Leaving the block with an exception releases
    the ones that do not belong to ``keep`` (the inputs); ``commit()`` hands them over instead."""

    def __init__(self, keep: Iterable[object] = ()) -> None:
        self._keep = {id(h) for h in keep}
        self.items: list = []

    def add(self, handle):
        self.items.append(handle)
        return handle

    def fresh(self) -> list:
        return [h for h in self.items if id(h) not in self._keep]

    def commit(self) -> tuple:
        out, self.items = tuple(self.items), []
        return out

    def __enter__(self) -> "_Staged":
        return self

    def __exit__(self, exc_type, exc, tb) -> bool:
        if exc_type is not None:
            _free(self.fresh())
        return False


def _duplicates(handles: Iterable[object]) -> tuple:
    """Deep copies of ``handles`` (distinct new objects), or nothing: a failed copy releases the
    copies made so far and re-raises."""

    sources = _distinct(handles, "copy sources")
    with _Staged(keep=sources) as staged:
        for h in sources:
            c = h.deep_copy()
            if c is None or any(c is x for x in sources) or any(c is x for x in staged.items):
                raise RuntimeError("deep_copy must return a new ciphertext object")
            staged.add(c)
        return staged.commit()


# ---------------------------------------------------------------------------- HBM page pool
class PooledCipher(Cipher):
    """A page ciphertext whose components are views into a KVPagePool slot; releasing the last
    of a slot's four ciphertexts returns the slot."""

    def __init__(self, cv, state, *, slots, batch_size, pool: "KVPagePool", slot: int):
        super().__init__(cv, state, slots=slots, batch_size=batch_size)
        self._pool = pool
        self._slot = int(slot)

    def release(self) -> None:
        if getattr(self, "_released", False):
            return
        super().release()
        self._pool._drop_ref(self._slot)

    def deep_copy(self) -> Cipher:
        return Cipher([u64_clone(c) for c in self.cv], self.state, slots=self.slots, batch_size=self.batch_size)


class KVPagePool:
    """Page slots of one layer in one HBM allocation: slot s holds the page's K0, K1, V0, V1 as
    ``buf[s][h][c]`` = [batch][limbs][N] (component c of handle h), limb-major like every ciphertext
    of this backend.  ``capacity`` bounds the pages resident at once (HBM: capacity x 8 x batch x
    limbs x N x 8 bytes)."""

    def __init__(self, ctx, limbs: int, capacity: int, batch: int = 1):
        if limbs < 1 or limbs > ctx.L or capacity < 1 or batch < 1:
            raise ValueError("pool needs 1 <= limbs <= L, capacity >= 1, batch >= 1")
        self.ctx = ctx
        self.limbs = int(limbs)
        self.capacity = int(capacity)
        self.batch = int(batch)
        self.buf = torch.empty((self.capacity, _HANDLES, 2, self.batch, self.limbs, ctx.N), dtype=torch.uint64,
                               device=ctx.device)
        self._free = list(range(self.capacity - 1, -1, -1))
        self._refs = [0] * self.capacity
        # per slot: the component views and the device address of every (handle, component, item)
        # polynomial, computed once so that an append does no tensor indexing
        poly = self.limbs * ctx.N * 8
        base = self.buf.data_ptr()
        self._views = [[(self.buf[s, h, 0], self.buf[s, h, 1]) for h in range(_HANDLES)] for s in range(self.capacity)]
        self._addr = [[base + (((s * _HANDLES + h) * 2 + c) * self.batch + b) * poly
                       for h in range(_HANDLES) for c in range(2) for b in range(self.batch)]
                      for s in range(self.capacity)]

    @property
    def nbytes(self) -> int:
        return int(self.buf.numel()) * 8

    @property
    def free_slots(self) -> int:
        return len(self._free)

    def _alloc(self) -> int:
        if not self._free:
            raise MemoryError(f"KV page pool exhausted ({self.capacity} slots of {self.slot_bytes} bytes)")
        s = self._free.pop()
        self._refs[s] = _HANDLES
        return s

    @property
    def slot_bytes(self) -> int:
        return _HANDLES * 2 * self.batch * self.limbs * self.ctx.N * 8

    def _drop_ref(self, s: int) -> None:
        self._refs[s] -= 1
        if self._refs[s] == 0:
            self._free.append(s)

    def _ciphers(self, s: int, template: Cipher) -> tuple:
        state = template.state.replace(cur_limbs=self.limbs)
        return tuple(PooledCipher(list(self._views[s][h]), state, slots=template.slots, batch_size=self.batch, pool=self,
                                  slot=s) for h in range(_HANDLES))

    def _item_addresses(self, handles) -> list:
        """Device address of every (handle, component, item) polynomial of ``handles``, in the pool's
        slot order, after one check per component tensor: uint64 on the pool's device, [batch][>=
        limbs][N] with contiguous limbs."""

        N, dev = self.ctx.N, self.buf.device
        out = []
        for h in handles:
            for t in h.cv:
                if (t.dtype != torch.uint64 or t.device != dev or t.dim() != 3 or t.shape[0] != self.batch
                        or t.shape[1] < self.limbs or t.shape[2] != N or t.stride(2) != 1 or t.stride(1) != N):
                    raise ValueError("page ciphertext components must be [batch][>= limbs][N] uint64 tensors with "
                                     "contiguous limbs on the pool's device")
                p0, sb = t.data_ptr(), t.stride(0) * 8
                out.extend(p0 + b * sb for b in range(self.batch))
        return out

    def fits(self, handles) -> bool:
        """True when every handle is a two-component ciphertext of this backend at the pool's level
        and batch (the fused path applies)."""

        for h in handles:
            if not isinstance(h, Cipher) or h.is_ext or len(h.cv) != 2:
                return False
            if int(h.state.cur_limbs) != self.limbs or int(h.batch_size) != self.batch:
                return False
        return True

    def add_pages(self, left, right) -> tuple:
        """The four sums left[h] + right[h] in a fresh slot, one hck_lincomb launch (8 * batch
        polynomial sums); both operands unchanged."""

        from . import fhe

        for a, b in zip(left, right):
            if int(a.state.scale_degree) != int(b.state.scale_degree) or not fhe._same_scale(
                    float(a.state.scaling_factor), float(b.state.scaling_factor)):
                raise ValueError("page and token differ in scale")
        lp, rp = self._item_addresses(left), self._item_addresses(right)
        s = self._alloc()
        try:
            ins = [a for pair in zip(lp, rp) for a in pair]
            self.ctx.lincomb_ptrs(ins, self.limbs, self._addr[s], 2)
        except BaseException:
            self._refs[s] = 0
            self._free.append(s)
            raise
        return self._ciphers(s, left[0])


# ---------------------------------------------------------------------------- ownership types
class _QuadOwner:
    """Shared behaviour of a token write and a page: four ciphertexts (two key groups, then two
    value groups) owned until they are released or moved out.  Subclasses are dataclasses with the
    fields ``key_groups`` and ``value_groups`` and define ``_rebuild(keys, values)``."""

    _noun = "ciphertext owner"

    def _own(self) -> None:
        self.key_groups = _groups(self.key_groups, "key_groups")
        self.value_groups = _groups(self.value_groups, "value_groups")
        _distinct(self.handles, self._noun)

    @property
    def handles(self) -> tuple:
        return (*self.key_groups, *self.value_groups)

    @property
    def is_released(self) -> bool:
        return self._released

    def _check_live(self) -> None:
        if self._released:
            raise RuntimeError(f"this {self._noun} no longer owns its ciphertexts (released or moved)")

    def _surrender(self) -> tuple:
        """Give the handles to the caller; this owner is empty afterwards."""

        self._check_live()
        out = self.handles
        self.key_groups = self.value_groups = ()
        self._released = True
        return out

    def clone(self):
        self._check_live()
        copies = _duplicates(self.handles)
        try:
            return self._rebuild(copies[:PAIRFOLD_GROUP_COUNT], copies[PAIRFOLD_GROUP_COUNT:])
        except BaseException:
            _free(copies)
            raise

    def release(self) -> None:
        if not self._released:
            failure = _free(self._surrender())
            if failure is not None:
                raise failure


@dataclass
class PairFoldTokenWrite(_QuadOwner):
    """The owned K/V payload of one token column: two key and two value ciphertexts."""

    key_groups: tuple | list
    value_groups: tuple | list
    column: int
    _released: bool = field(default=False, init=False, repr=False)
    _noun = "token write"

    def __post_init__(self) -> None:
        self.column = int(self.column)
        if self.column not in range(PAIRFOLD_PAGE_SIZE):
            raise ValueError(f"column {self.column} is not a page column (0..{PAIRFOLD_PAGE_SIZE - 1})")
        self._own()

    @property
    def is_consumed(self) -> bool:
        return self._released

    def _rebuild(self, keys, values) -> "PairFoldTokenWrite":
        return PairFoldTokenWrite(keys, values, self.column)

    def move(self) -> "PairFoldTokenWrite":
        """A new write owning these handles; this one is consumed (no copy)."""

        self._check_live()
        successor = self._rebuild(self.key_groups, self.value_groups)
        self._surrender()
        return successor


@dataclass
class PairFoldCipherPage(_QuadOwner):
    """One page: two K and two V ciphertexts holding ``occupied`` of its 128 token columns."""

    key_groups: tuple | list
    value_groups: tuple | list
    occupied: int
    _released: bool = field(default=False, init=False, repr=False)
    _noun = "PairFold page"

    def __post_init__(self) -> None:
        self.occupied = int(self.occupied)
        if not 0 < self.occupied <= PAIRFOLD_PAGE_SIZE:
            raise ValueError(f"occupied count {self.occupied} is outside 1..{PAIRFOLD_PAGE_SIZE}")
        self._own()

    @property
    def remaining(self) -> int:
        return PAIRFOLD_PAGE_SIZE - self.occupied

    def _rebuild(self, keys, values) -> "PairFoldCipherPage":
        return PairFoldCipherPage(keys, values, self.occupied)

    @classmethod
    def from_token_write(cls, token: PairFoldTokenWrite, occupied: int) -> "PairFoldCipherPage":
        """The token's handles become the page; the token is consumed only after the page has
        been built (a bad ``occupied`` leaves the token untouched)."""

        if not isinstance(token, PairFoldTokenWrite):
            raise TypeError(f"expected a PairFoldTokenWrite, got {type(token).__name__}")
        token._check_live()
        page = cls(token.key_groups, token.value_groups, occupied)
        token._surrender()
        return page


@dataclass
class PairFoldLayerCache:
    """Append-only page list of one layer; every page but the last is full.  ``pool`` (optional)
    holds the pages this cache creates by addition."""

    pages: tuple | list = ()
    content_tokens: int = 0
    layout_tag: str = PAIRFOLD_LAYOUT_TAG
    pool: KVPagePool | None = field(default=None, repr=False)
    _released: bool = field(default=False, init=False, repr=False)

    def __post_init__(self) -> None:
        self.pages = tuple(self.pages)
        self.content_tokens = int(self.content_tokens)
        self.layout_tag = str(self.layout_tag)
        self._check_shape()

    @property
    def is_released(self) -> bool:
        return self._released

    @property
    def occupied(self) -> int:
        return self.content_tokens

    @property
    def handles(self) -> tuple:
        self._check_live()
        return tuple(h for page in self.pages for h in page.handles)

    def _check_live(self) -> None:
        if self._released:
            raise RuntimeError("this PairFold layer cache was released")

    def _check_shape(self) -> None:
        """Layout tag, page types, full pages before the tail, token count, no shared handle."""

        if self.layout_tag != PAIRFOLD_LAYOUT_TAG:
            raise ValueError(f"unknown layout tag {self.layout_tag!r} (this cache is {PAIRFOLD_LAYOUT_TAG!r})")
        if self.content_tokens < 0:
            raise ValueError(f"content_tokens {self.content_tokens} is negative")
        for page in self.pages:
            if not isinstance(page, PairFoldCipherPage):
                raise TypeError(f"pages hold PairFoldCipherPage objects, not {type(page).__name__}")
            page._check_live()
        if any(p.occupied != PAIRFOLD_PAGE_SIZE for p in self.pages[:-1]):
            raise ValueError("a page before the last one is not full")
        counted = sum(p.occupied for p in self.pages)
        if counted != self.content_tokens:
            raise ValueError(f"content_tokens is {self.content_tokens} but the pages hold {counted} tokens")
        _distinct(self.handles, "PairFold layer cache")

    def _next_column(self) -> int:
        """The column the next token must carry: 0 opens a page, else the tail's first free one."""

        if not self.pages or self.pages[-1].remaining == 0:
            return 0
        return self.pages[-1].occupied

    def clone(self) -> "PairFoldLayerCache":
        self._check_live()
        self._check_shape()
        copies = _duplicates(self.handles)
        try:
            pages, at = [], 0
            for page in self.pages:
                quad = copies[at:at + _HANDLES]
                pages.append(PairFoldCipherPage(quad[:PAIRFOLD_GROUP_COUNT], quad[PAIRFOLD_GROUP_COUNT:], page.occupied))
                at += _HANDLES
            return PairFoldLayerCache(pages=pages, content_tokens=self.content_tokens, layout_tag=self.layout_tag,
                                      pool=self.pool)
        except BaseException:
            _free(copies)
            raise

    def extend_pages(self, other: "PairFoldLayerCache") -> None:
        """Move the pages of ``other`` (a prefill's output) behind this cache's full tail, no copy;
        ``other`` ends released and empty."""

        self._check_live()
        if not isinstance(other, PairFoldLayerCache):
            raise TypeError(f"expected a PairFoldLayerCache, got {type(other).__name__}")
        if other is self:
            raise ValueError("a cache cannot take its own pages")
        other._check_live()
        self._check_shape()
        other._check_shape()
        if not other.pages:
            return
        if self._next_column() != 0:
            raise ValueError("the tail must be full before another cache's pages can follow it")
        _distinct(self.handles + other.handles, "joined PairFold caches")
        self.pages += other.pages
        self.content_tokens += other.content_tokens
        other.pages, other.content_tokens, other._released = (), 0, True

    def _sums(self, tail: PairFoldCipherPage, token: PairFoldTokenWrite, crypto_context, staged: _Staged) -> None:
        """The four page + token sums into ``staged``: one fused launch into a pool slot when the
        pool fits them, else one homo_add per ciphertext (the reference's path)."""

        pairs = tuple(zip(tail.handles, token.handles))
        if self.pool is not None and self.pool.fits(tail.handles + token.handles):
            for out in self.pool.add_pages(tail.handles, token.handles):
                staged.add(out)
            return
        for page_ct, token_ct in pairs:
            staged.add(crypto_context.fhe.homo_add(page_ct, token_ct, crypto_context.context))

    def append(self, token: PairFoldTokenWrite, *, crypto_context) -> tuple[int, int]:
        """Consume ``token`` into its column; returns (page index, column).  A token at column 0
        becomes a new page by move; any other column is added into the tail, and the four sums
        replace the tail only once all of them exist (then the old tail and the token are
        released).  Anything that fails first leaves the cache and the token as they were."""

        self._check_live()
        self._check_shape()
        if not isinstance(token, PairFoldTokenWrite):
            raise TypeError(f"expected a PairFoldTokenWrite, got {type(token).__name__}")
        token._check_live()
        _distinct(self.handles + token.handles, "cache and token write")
        column = self._next_column()
        if token.column != column:
            raise ValueError(f"token column {token.column} is not the next free column {column}")
        if column == 0:
            self.pages += (PairFoldCipherPage.from_token_write(token, occupied=1),)
            self.content_tokens += 1
            return len(self.pages) - 1, 0
        tail = self.pages[-1]
        inputs = self.handles + token.handles
        with _Staged(keep=inputs) as staged:
            self._sums(tail, token, crypto_context, staged)
            _distinct(staged.items, "sums of an append")
            if len(staged.fresh()) != len(staged.items):
                raise ValueError("homo_add returned one of its inputs: outputs must be new ciphertexts (alias)")
            sums = staged.items
            grown = PairFoldCipherPage(sums[:PAIRFOLD_GROUP_COUNT], sums[PAIRFOLD_GROUP_COUNT:], tail.occupied + 1)
            staged.commit()
        self.pages = self.pages[:-1] + (grown,)
        self.content_tokens += 1
        failure = _free(tail._surrender() + token._surrender())
        if failure is not None:
            raise failure
        return len(self.pages) - 1, column

    def release(self) -> None:
        if self._released:
            return
        pages = self.pages
        self.pages, self.content_tokens, self._released = (), 0, True
        failures = []
        for page in pages:
            try:
                page.release()
            except BaseException as exc:
                failures.append(exc)
        if failures:
            raise failures[0]


def drop_pairfold_token_to_limbs(token: PairFoldTokenWrite, *, target_limbs: int, crypto_context,
                                 bootstrap_operator=None, bootstrap_iterations: int = 1,
                                 value_target_limbs: int | None = None) -> PairFoldTokenWrite:
    """A write whose K0, K1 sit at ``target_limbs`` and V0, V1 at ``value_target_limbs`` (default
    the same), limbs dropped by ``fhe.align_to``; a ciphertext with fewer limbs than its target is
    refreshed by ``bootstrap_operator.refresh`` first (llama3fhe/operators/pairfold_kv_cache.py:
    478-621).  All four results exist before ``token`` is consumed; a failure releases only what
    this call created.  A token already at its targets is moved, not copied."""

    if not isinstance(token, PairFoldTokenWrite):
        raise TypeError(f"expected a PairFoldTokenWrite, got {type(token).__name__}")
    token._check_live()
    key_t = int(target_limbs)
    val_t = key_t if value_target_limbs is None else int(value_target_limbs)
    if min(key_t, val_t) < 2:
        raise ValueError(f"limb targets {key_t} / {val_t}: a dropped ciphertext keeps at least two limbs")
    if int(bootstrap_iterations) < 1:
        raise ValueError(f"bootstrap_iterations is {bootstrap_iterations}; it must be at least 1")
    sources = token.handles
    targets = (key_t,) * PAIRFOLD_GROUP_COUNT + (val_t,) * PAIRFOLD_GROUP_COUNT
    for ct in sources:
        if bool(ct.is_ext) or int(ct.state.scale_degree) != 1:
            raise ValueError("limb drops take non-extended ciphertexts of scale degree 1")
    current = tuple(int(ct.state.cur_limbs) for ct in sources)
    if bootstrap_operator is None:
        for have, want in zip(current, targets):
            if have < want:
                raise ValueError(f"a page at {have} limbs needs a refresh to reach {want}, and no refresh operator was given")
    if current == targets:
        return token.move()
    ops = getattr(crypto_context, "fhe", None)
    if ops is None:
        from . import fhe as ops
    native = getattr(crypto_context, "context", crypto_context)
    with _Staged(keep=sources) as staged:
        for ct, have, want in zip(sources, current, targets):
            refreshed = None
            if have < want:
                refreshed = bootstrap_operator.refresh(ct, iterations=int(bootstrap_iterations))
                if any(refreshed is x for x in sources):
                    raise RuntimeError("bootstrap refresh returned its input; it must return a new ciphertext")
            base = ct if refreshed is None else refreshed
            try:
                staged.add(ops.align_to(base, base.state.replace(cur_limbs=want), native))
            finally:
                if refreshed is not None:
                    _free([refreshed])
        if len(staged.fresh()) != len(staged.items):
            raise RuntimeError("align_to returned one of the token's ciphertexts (alias)")
        _distinct(staged.items, "limb-drop results")
        result = PairFoldTokenWrite(staged.items[:PAIRFOLD_GROUP_COUNT], staged.items[PAIRFOLD_GROUP_COUNT:],
                                    token.column)
        staged.commit()
    try:
        token.release()
    except BaseException:
        _free(result.handles)
        raise
    return result
