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


# ---------------------------------------------------------------------------- handle helpers
def _group(values: Iterable[object], name: str) -> tuple:
    g = tuple(values)
    if len(g) != PAIRFOLD_GROUP_COUNT:
        raise ValueError(f"{name} must contain exactly {PAIRFOLD_GROUP_COUNT} ciphertexts, got {len(g)}")
    if any(v is None for v in g):
        raise ValueError(f"{name} must not contain None")
    return g


def _unique(handles: Iterable[object], owner: str) -> None:
    hs = tuple(handles)
    if len({id(h) for h in hs}) != len(hs):
        raise ValueError(f"{owner}: ciphertext handles must not alias")


def _release_all(handles: Iterable[object]) -> BaseException | None:
    """Release every distinct handle once; return the first error after trying them all."""

    first = None
    seen: set[int] = set()
    for h in tuple(handles):
        if id(h) in seen:
            continue
        seen.add(id(h))
        try:
            rel = getattr(h, "release", None)
            if callable(rel):
                rel()
        except BaseException as err:  # every handle is still tried
            if first is None:
                first = err
    return first


def _deep_copies(handles: Iterable[object]) -> tuple:
    src = tuple(handles)
    _unique(src, "clone sources")
    src_ids = {id(h) for h in src}
    made: list = []
    try:
        for h in src:
            c = h.deep_copy()
            if c is None:
                raise RuntimeError("ciphertext deep_copy returned None")
            if id(c) in src_ids:
                raise RuntimeError("ciphertext deep_copy must not return a source handle")
            if any(c is m for m in made):
                raise RuntimeError("ciphertext deep_copy outputs must not alias each other")
            made.append(c)
    except BaseException:
        _release_all(m for m in made if id(m) not in src_ids)
        raise
    return tuple(made)


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
        return tuple(PooledCipher([self.buf[s, h, 0], self.buf[s, h, 1]], template.state.replace(cur_limbs=self.limbs),
                                  slots=template.slots, batch_size=self.batch, pool=self, slot=s)
                     for h in range(_HANDLES))

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
        s = self._alloc()
        try:
            xs, outs = [], []
            for h in range(_HANDLES):
                for c in range(2):
                    for b in range(self.batch):
                        xs.append([left[h].cv[c][b], right[h].cv[c][b]])
                        outs.append(self.buf[s, h, c, b])
            self.ctx.lincomb(xs, self.limbs, outs)
        except BaseException:
            self._refs[s] = 0
            self._free.append(s)
            raise
        return self._ciphers(s, left[0])


# ---------------------------------------------------------------------------- ownership types
@dataclass
class PairFoldTokenWrite:
    """The owned K/V payload of one token column: two key and two value ciphertexts."""

    key_groups: tuple | list
    value_groups: tuple | list
    column: int
    _released: bool = field(default=False, init=False, repr=False)

    def __post_init__(self) -> None:
        self.key_groups = _group(self.key_groups, "key_groups")
        self.value_groups = _group(self.value_groups, "value_groups")
        self.column = int(self.column)
        if not 0 <= self.column < PAIRFOLD_PAGE_SIZE:
            raise ValueError(f"column must be in [0, {PAIRFOLD_PAGE_SIZE - 1}], got {self.column}")
        _unique(self.handles, "token write")

    @property
    def handles(self) -> tuple:
        return tuple(self.key_groups) + tuple(self.value_groups)

    @property
    def is_released(self) -> bool:
        return bool(self._released)

    is_consumed = is_released

    def _check_live(self) -> None:
        if self._released:
            raise RuntimeError("PairFold token write has already been consumed")

    def _take(self) -> tuple:
        """Give up ownership without releasing (the caller now owns the handles)."""

        self._check_live()
        owned = self.handles
        self.key_groups, self.value_groups = (), ()
        self._released = True
        return owned

    def clone(self) -> "PairFoldTokenWrite":
        self._check_live()
        copies = _deep_copies(self.handles)
        try:
            return PairFoldTokenWrite(copies[:PAIRFOLD_GROUP_COUNT], copies[PAIRFOLD_GROUP_COUNT:], self.column)
        except BaseException:
            _release_all(copies)
            raise

    def move(self) -> "PairFoldTokenWrite":
        self._check_live()
        moved = PairFoldTokenWrite(self.key_groups, self.value_groups, self.column)  # validates first
        self._take()
        return moved

    def release(self) -> None:
        if self._released:
            return
        err = _release_all(self._take())
        if err is not None:
            raise err


@dataclass
class PairFoldCipherPage:
    """One page: two K and two V ciphertexts holding ``occupied`` of its 128 token columns."""

    key_groups: tuple | list
    value_groups: tuple | list
    occupied: int
    _released: bool = field(default=False, init=False, repr=False)

    def __post_init__(self) -> None:
        self.key_groups = _group(self.key_groups, "key_groups")
        self.value_groups = _group(self.value_groups, "value_groups")
        self.occupied = int(self.occupied)
        if not 1 <= self.occupied <= PAIRFOLD_PAGE_SIZE:
            raise ValueError(f"occupied must be in [1, {PAIRFOLD_PAGE_SIZE}], got {self.occupied}")
        _unique(self.handles, "PairFold page")

    @property
    def handles(self) -> tuple:
        return tuple(self.key_groups) + tuple(self.value_groups)

    @property
    def remaining(self) -> int:
        return PAIRFOLD_PAGE_SIZE - self.occupied

    @property
    def is_released(self) -> bool:
        return bool(self._released)

    def _check_live(self) -> None:
        if self._released:
            raise RuntimeError("PairFold page has already been released")

    def _take(self) -> tuple:
        self._check_live()
        owned = self.handles
        self.key_groups, self.value_groups = (), ()
        self._released = True
        return owned

    @classmethod
    def from_token_write(cls, token: PairFoldTokenWrite, occupied: int) -> "PairFoldCipherPage":
        """The token's handles become the page (no copy); the token is consumed only once the page
        has been built and validated."""

        if not isinstance(token, PairFoldTokenWrite):
            raise TypeError("token must be a PairFoldTokenWrite")
        token._check_live()
        page = cls(key_groups=token.key_groups, value_groups=token.value_groups, occupied=occupied)
        token._take()
        return page

    def clone(self) -> "PairFoldCipherPage":
        self._check_live()
        copies = _deep_copies(self.handles)
        try:
            return PairFoldCipherPage(copies[:PAIRFOLD_GROUP_COUNT], copies[PAIRFOLD_GROUP_COUNT:], self.occupied)
        except BaseException:
            _release_all(copies)
            raise

    def release(self) -> None:
        if self._released:
            return
        err = _release_all(self._take())
        if err is not None:
            raise err


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
        self._validate()

    @property
    def is_released(self) -> bool:
        return bool(self._released)

    @property
    def occupied(self) -> int:
        return self.content_tokens

    @property
    def handles(self) -> tuple:
        self._check_live()
        return tuple(h for p in self.pages for h in p.handles)

    def _check_live(self) -> None:
        if self._released:
            raise RuntimeError("PairFold layer cache has already been released")

    def _validate(self) -> None:
        if self.layout_tag != PAIRFOLD_LAYOUT_TAG:
            raise ValueError(f"layout_tag must be {PAIRFOLD_LAYOUT_TAG!r}, got {self.layout_tag!r}")
        if self.content_tokens < 0:
            raise ValueError("content_tokens must be non-negative")
        if not self.pages:
            if self.content_tokens:
                raise ValueError("an empty PairFold cache must hold zero tokens")
            return
        total = 0
        for i, p in enumerate(self.pages):
            if not isinstance(p, PairFoldCipherPage):
                raise TypeError("pages must be PairFoldCipherPage objects")
            p._check_live()
            if i < len(self.pages) - 1 and p.occupied != PAIRFOLD_PAGE_SIZE:
                raise ValueError("every page but the tail must be full")
            total += p.occupied
        if total != self.content_tokens:
            raise ValueError(f"content_tokens {self.content_tokens} differs from the pages' occupancy {total}")
        _unique([h for p in self.pages for h in p.handles], "PairFold cache")

    def clone(self) -> "PairFoldLayerCache":
        self._check_live()
        self._validate()
        copies = _deep_copies(self.handles)
        try:
            pages = tuple(PairFoldCipherPage(copies[i * _HANDLES:i * _HANDLES + PAIRFOLD_GROUP_COUNT],
                                             copies[i * _HANDLES + PAIRFOLD_GROUP_COUNT:(i + 1) * _HANDLES],
                                             p.occupied) for i, p in enumerate(self.pages))
            return PairFoldLayerCache(pages=pages, content_tokens=self.content_tokens, layout_tag=self.layout_tag,
                                      pool=self.pool)
        except BaseException:
            _release_all(copies)
            raise

    def extend_pages(self, other: "PairFoldLayerCache") -> None:
        """Move the pages of ``other`` (prefill output) behind this cache's full tail, no copy."""

        self._check_live()
        if not isinstance(other, PairFoldLayerCache):
            raise TypeError("other must be a PairFoldLayerCache")
        other._check_live()
        if other is self:
            raise ValueError("cannot extend a cache with itself")
        self._validate()
        other._validate()
        if not other.pages:
            return
        if self.pages and self.pages[-1].occupied != PAIRFOLD_PAGE_SIZE:
            raise ValueError("the tail must be full before pages are appended")
        _unique(self.handles + other.handles, "combined PairFold cache")
        self.pages = self.pages + other.pages
        self.content_tokens += other.content_tokens
        other.pages, other.content_tokens, other._released = (), 0, True

    def append(self, token: PairFoldTokenWrite, *, crypto_context) -> tuple[int, int]:
        """Consume ``token`` into its column; returns (page index, column).  A new page takes the
        token's handles; a partial tail gets the four sums (fused into a pool slot when the cache
        has a pool that fits, else four ``crypto_context.fhe.homo_add`` calls), committed together."""

        self._check_live()
        self._validate()
        if not isinstance(token, PairFoldTokenWrite):
            raise TypeError("token must be a PairFoldTokenWrite")
        token._check_live()
        mine = tuple(h for p in self.pages for h in p.handles)
        _unique(mine + token.handles, "cache and token write")
        opens = not self.pages or self.pages[-1].occupied == PAIRFOLD_PAGE_SIZE
        want = 0 if opens else self.pages[-1].occupied
        if token.column != want:
            raise ValueError(f"token column must be {want}, got {token.column}")
        if opens:
            self.pages = self.pages + (PairFoldCipherPage.from_token_write(token, occupied=1),)
            self.content_tokens += 1
            return len(self.pages) - 1, 0

        tail = self.pages[-1]
        inputs = {id(h) for h in mine + token.handles}
        sums: list = []
        try:
            if self.pool is not None and self.pool.fits(tail.handles + token.handles):
                sums = list(self.pool.add_pages(tail.handles, token.handles))
            else:
                for a, b in zip(tail.handles, token.handles):
                    sums.append(crypto_context.fhe.homo_add(a, b, crypto_context.context))
            _unique(sums, "append outputs")
            if any(id(s) in inputs for s in sums):
                raise ValueError("homo_add outputs must not alias their inputs")
            page = PairFoldCipherPage(tuple(sums[:PAIRFOLD_GROUP_COUNT]), tuple(sums[PAIRFOLD_GROUP_COUNT:]),
                                      tail.occupied + 1)
        except BaseException:
            _release_all(s for s in sums if id(s) not in inputs)
            raise
        # commit, then release the replaced tail and the token
        self.pages = self.pages[:-1] + (page,)
        self.content_tokens += 1
        err = _release_all(tail._take() + token._take())
        if err is not None:
            raise err
        return len(self.pages) - 1, want

    def release(self) -> None:
        if self._released:
            return
        pages = self.pages
        self.pages, self.content_tokens, self._released = (), 0, True
        first = None
        for p in pages:
            try:
                p.release()
            except BaseException as err:
                if first is None:
                    first = err
        if first is not None:
            raise first


def drop_pairfold_token_to_limbs(token: PairFoldTokenWrite, *, target_limbs: int, crypto_context,
                                 bootstrap_operator=None, bootstrap_iterations: int = 1,
                                 value_target_limbs: int | None = None) -> PairFoldTokenWrite:
    """Bring K0, K1 to ``target_limbs`` and V0, V1 to ``value_target_limbs`` (default the same):
    drop limbs, or refresh first with ``bootstrap_operator.refresh`` when a ciphertext has fewer
    limbs than its target.  All four replacements are built before ``token`` is consumed; any
    failure releases only the new ciphertexts (pairfold_kv_cache.py:478-621)."""

    if not isinstance(token, PairFoldTokenWrite):
        raise TypeError("token must be a PairFoldTokenWrite")
    token._check_live()
    target_limbs = int(target_limbs)
    vt = target_limbs if value_target_limbs is None else int(value_target_limbs)
    if target_limbs <= 1 or vt <= 1:
        raise ValueError(f"a modulus drop must leave more than one limb, got {target_limbs} / {vt}")
    iters = int(bootstrap_iterations)
    if iters <= 0:
        raise ValueError(f"bootstrap_iterations must be positive, got {iters}")
    inputs = token.handles
    targets = (target_limbs,) * PAIRFOLD_GROUP_COUNT + (vt,) * PAIRFOLD_GROUP_COUNT
    for c in inputs:
        if int(c.state.scale_degree) != 1 or bool(c.is_ext):
            raise ValueError("modulus-only scheduling requires non-extended degree-1 ciphertexts")
    have = tuple(int(c.state.cur_limbs) for c in inputs)
    short = [(h, t) for h, t in zip(have, targets) if h < t]
    if short and bootstrap_operator is None:
        raise ValueError(f"too few limbs for the drop: {short[0][0]} < {short[0][1]}")
    if have == targets:
        return token.move()
    fhe = getattr(crypto_context, "fhe", None)
    ctx = getattr(crypto_context, "context", crypto_context)
    if fhe is None:
        from . import fhe
    ids = {id(c) for c in inputs}
    made: list = []
    try:
        for c, h, t in zip(inputs, have, targets):
            work, fresh = c, None
            if h < t:
                fresh = bootstrap_operator.refresh(c, iterations=iters)
                if id(fresh) in ids:
                    raise RuntimeError("bootstrap refresh must return a new ciphertext")
                work = fresh
            try:
                made.append(fhe.align_to(work, work.state.replace(cur_limbs=t), ctx))
            finally:
                if fresh is not None:
                    _release_all([fresh])
        _unique(made, "limb-drop outputs")
        if any(id(m) in ids for m in made):
            raise RuntimeError("limb-drop outputs must not alias the token's ciphertexts")
        out = PairFoldTokenWrite(made[:PAIRFOLD_GROUP_COUNT], made[PAIRFOLD_GROUP_COUNT:], token.column)
    except BaseException:
        _release_all(m for m in made if id(m) not in ids)
        raise
    made = []
    try:
        token.release()
    except BaseException:
        _release_all(out.handles)
        raise
    return out
