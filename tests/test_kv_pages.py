"""CPU tests of the PairFold KV cache ownership rules (fake ciphertexts; no GPU): the behaviours
llama3fhe's own tests pin for pairfold_kv_cache.py (tests/test_pairfold_kv_cache.py) -- moves
without copies, the four-sum transactional append and its rollback at every add, the column rule,
deep clones, idempotent release, and the invariants."""

from __future__ import annotations

import pytest

from holmes_amd.kv_pages import (
    PAIRFOLD_LAYOUT_TAG,
    PAIRFOLD_PAGE_SIZE,
    PairFoldCipherPage,
    PairFoldLayerCache,
    PairFoldTokenWrite,
    drop_pairfold_token_to_limbs,
)


class Fake:
    """A ciphertext stand-in: a value, copy and release counters."""

    def __init__(self, value, label, copier=None, limbs=6):
        self.value, self.label, self.copier = int(value), label, copier
        self.copies = 0
        self.releases = 0
        self.state = _State(limbs)
        self.is_ext = False

    def deep_copy(self):
        self.copies += 1
        if self.copier is not None:
            return self.copier(self)
        return Fake(self.value, self.label + "'")

    def release(self):
        assert self.releases == 0, f"released twice: {self.label}"
        self.releases = 1


class _State:
    def __init__(self, limbs, scale_degree=1):
        self.cur_limbs, self.scale_degree = limbs, scale_degree

    def replace(self, **kw):
        s = _State(self.cur_limbs, self.scale_degree)
        for k, v in kw.items():
            setattr(s, k, v)
        return s


class FakeFhe:
    def __init__(self, ctx, fail_at=None):
        self.ctx, self.fail_at, self.calls, self.outputs = ctx, fail_at, [], []

    def homo_add(self, a, b, ctx):
        assert ctx is self.ctx
        i = len(self.calls)
        self.calls.append((a, b))
        if i == self.fail_at:
            raise RuntimeError(f"add failed at {i}")
        out = Fake(a.value + b.value, f"sum{i}")
        self.outputs.append(out)
        return out

    def align_to(self, c, state, ctx):
        out = Fake(c.value, c.label + ".drop", limbs=state.cur_limbs)
        return out


class FakeContext:
    def __init__(self, fail_at=None):
        self.context = object()
        self.fhe = FakeFhe(self.context, fail_at)


def _four(label, start, copier=None):
    return [Fake(start + i, f"{label}{i}", copier) for i in range(4)]


def token(column, label="t", start=100, copier=None):
    h = _four(label, start, copier)
    return PairFoldTokenWrite(h[:2], h[2:], column)


def page(occupied, label="p", start=10, copier=None):
    h = _four(label, start, copier)
    return PairFoldCipherPage(h[:2], h[2:], occupied)


def same(a, b):
    a, b = tuple(a), tuple(b)
    return len(a) == len(b) and all(x is y for x, y in zip(a, b))


def test_first_append_moves_the_token_without_work():
    cache = PairFoldLayerCache()
    t = token(0)
    hs = t.handles
    ctx = FakeContext()
    assert cache.append(t, crypto_context=ctx) == (0, 0)
    assert cache.layout_tag == PAIRFOLD_LAYOUT_TAG and cache.content_tokens == 1
    assert same(cache.pages[0].handles, hs) and t.is_consumed and not t.key_groups
    assert ctx.fhe.calls == [] and all(h.copies == 0 and h.releases == 0 for h in hs)


@pytest.mark.parametrize("occupied", [1, PAIRFOLD_PAGE_SIZE])
def test_page_from_token_moves_and_releases_once(occupied):
    t = token(0)
    hs = t.handles
    p = PairFoldCipherPage.from_token_write(t, occupied)
    assert t.is_consumed and same(p.handles, hs) and p.occupied == occupied
    p.release()
    p.release()
    assert all(h.releases == 1 for h in hs)


@pytest.mark.parametrize("occupied", [0, PAIRFOLD_PAGE_SIZE + 1])
def test_page_from_token_rejects_bad_occupancy_atomically(occupied):
    t = token(0)
    hs = t.handles
    with pytest.raises(ValueError, match="occupied"):
        PairFoldCipherPage.from_token_write(t, occupied)
    assert not t.is_consumed and same(t.handles, hs) and all(h.releases == 0 for h in hs)


def test_full_tail_opens_a_new_page_and_history_is_untouched():
    hist = page(PAIRFOLD_PAGE_SIZE, "h")
    cache = PairFoldLayerCache(pages=(hist,), content_tokens=PAIRFOLD_PAGE_SIZE)
    t = token(0)
    hs = t.handles
    ctx = FakeContext()
    assert cache.append(t, crypto_context=ctx) == (1, 0)
    assert cache.pages[0] is hist and same(cache.pages[1].handles, hs) and ctx.fhe.calls == []
    assert cache.content_tokens == PAIRFOLD_PAGE_SIZE + 1


def test_partial_append_adds_four_and_commits():
    frozen, tail = page(PAIRFOLD_PAGE_SIZE, "f", 0), page(5, "tail", 20)
    cache = PairFoldLayerCache(pages=(frozen, tail), content_tokens=PAIRFOLD_PAGE_SIZE + 5)
    t = token(5, start=200)
    th, tk = tail.handles, t.handles
    ctx = FakeContext()
    assert cache.append(t, crypto_context=ctx) == (1, 5)
    assert [c for c in ctx.fhe.calls] == list(zip(th, tk))
    assert same(cache.pages[1].handles, ctx.fhe.outputs) and cache.pages[1].occupied == 6
    assert [o.value for o in ctx.fhe.outputs] == [a.value + b.value for a, b in zip(th, tk)]
    assert all(h.releases == 1 for h in th + tk) and all(h.releases == 0 for h in frozen.handles)
    assert cache.pages[0] is frozen and t.is_consumed and tail.is_released


@pytest.mark.parametrize("fail_at", range(4))
def test_failed_add_rolls_back(fail_at):
    tail = page(11, "tail", 20)
    cache = PairFoldLayerCache(pages=(tail,), content_tokens=11)
    t = token(11, start=200)
    th, tk = tail.handles, t.handles
    ctx = FakeContext(fail_at)
    with pytest.raises(RuntimeError, match=f"add failed at {fail_at}"):
        cache.append(t, crypto_context=ctx)
    assert cache.pages == (tail,) and cache.content_tokens == 11 and tail.occupied == 11
    assert same(tail.handles, th) and same(t.handles, tk) and not t.is_consumed
    assert all(h.releases == 0 for h in th + tk)
    assert len(ctx.fhe.outputs) == fail_at and all(o.releases == 1 for o in ctx.fhe.outputs)


@pytest.mark.parametrize("pages,tokens,bad", [((), 0, 1), ("partial", 7, 6), ("full", PAIRFOLD_PAGE_SIZE, 127)])
def test_wrong_column_is_rejected_before_any_work(pages, tokens, bad):
    if pages == "partial":
        pages = (page(7),)
    elif pages == "full":
        pages = (page(PAIRFOLD_PAGE_SIZE),)
    cache = PairFoldLayerCache(pages=pages, content_tokens=tokens)
    t = token(bad)
    ctx = FakeContext()
    with pytest.raises(ValueError, match="column"):
        cache.append(t, crypto_context=ctx)
    assert ctx.fhe.calls == [] and not t.is_consumed and cache.content_tokens == tokens


def test_column_127_fills_the_page_then_column_0_opens_the_next():
    cache = PairFoldLayerCache(pages=(page(127),), content_tokens=127)
    ctx = FakeContext()
    cache.append(token(127, "a", 200), crypto_context=ctx)
    assert len(cache.pages) == 1 and cache.pages[0].occupied == PAIRFOLD_PAGE_SIZE and len(ctx.fhe.calls) == 4
    full = cache.pages[0]
    cache.append(token(0, "b", 300), crypto_context=ctx)
    assert cache.pages[0] is full and cache.pages[1].occupied == 1 and len(ctx.fhe.calls) == 4


def test_extend_pages_moves_prefill_pages():
    hist, new = page(PAIRFOLD_PAGE_SIZE, "h"), page(3, "n", 20)
    a = PairFoldLayerCache(pages=(hist,), content_tokens=PAIRFOLD_PAGE_SIZE)
    b = PairFoldLayerCache(pages=(new,), content_tokens=3)
    a.extend_pages(b)
    assert a.pages == (hist, new) and a.content_tokens == PAIRFOLD_PAGE_SIZE + 3 and b.is_released
    partial = PairFoldLayerCache(pages=(page(127, "x"),), content_tokens=127)
    more = PairFoldLayerCache(pages=(page(1, "y"),), content_tokens=1)
    with pytest.raises(ValueError, match="tail must be full"):
        partial.extend_pages(more)  # the message names the rule: the tail must be full first
    assert not more.is_released and more.content_tokens == 1


def test_clones_are_deep_and_release_is_idempotent():
    t = token(37)
    c = t.clone()
    assert all(a is not b and a.value == b.value for a, b in zip(t.handles, c.handles))
    cache = PairFoldLayerCache(pages=(page(PAIRFOLD_PAGE_SIZE, "a"), page(9, "b", 30)),
                               content_tokens=PAIRFOLD_PAGE_SIZE + 9)
    cc = cache.clone()
    assert cc.content_tokens == cache.content_tokens
    assert all(x is not y for x, y in zip(cache.handles, cc.handles))
    hs = cache.handles
    cache.release()
    cache.release()
    assert all(h.releases == 1 for h in hs) and all(h.releases == 0 for h in cc.handles)
    with pytest.raises(RuntimeError):
        cache.append(token(9), crypto_context=FakeContext())
    with pytest.raises(RuntimeError):
        cache.clone()


def test_clone_failure_releases_only_the_partial_copies():
    made = []

    def copier(src):
        if len(made) == 2:
            raise RuntimeError("copy failed")
        out = Fake(src.value, src.label + "'")
        made.append(out)
        return out

    t = token(3, copier=copier)
    with pytest.raises(RuntimeError, match="copy failed"):
        t.clone()
    assert all(m.releases == 1 for m in made) and all(h.releases == 0 for h in t.handles)


def test_invariants_and_aliases_are_rejected():
    with pytest.raises(ValueError):
        token(PAIRFOLD_PAGE_SIZE)
    with pytest.raises(ValueError):
        PairFoldTokenWrite([Fake(1, "a")], [Fake(2, "b"), Fake(3, "c")], 0)
    x = Fake(1, "x")
    with pytest.raises(ValueError, match="alias"):
        PairFoldTokenWrite([x, x], [Fake(2, "b"), Fake(3, "c")], 0)
    with pytest.raises(ValueError):
        PairFoldLayerCache(pages=(page(5), page(5, "q", 40)), content_tokens=10)  # non-tail page not full
    with pytest.raises(ValueError):
        PairFoldLayerCache(pages=(page(5),), content_tokens=6)
    with pytest.raises(ValueError):
        PairFoldLayerCache(layout_tag="other")
    p = page(PAIRFOLD_PAGE_SIZE)
    q = PairFoldCipherPage(p.key_groups, [Fake(7, "v0"), Fake(8, "v1")], 3)
    with pytest.raises(ValueError, match="alias"):
        PairFoldLayerCache(pages=(p, q), content_tokens=PAIRFOLD_PAGE_SIZE + 3)


def test_limb_drop_is_transactional():
    ctx = FakeContext()
    t = token(4)
    hs0 = t.handles
    same_level = drop_pairfold_token_to_limbs(t, target_limbs=6, crypto_context=ctx)  # at target: a move
    assert t.is_consumed and same(same_level.handles, hs0) and all(h.copies == 0 for h in hs0)
    hs = same_level.handles
    dropped = drop_pairfold_token_to_limbs(same_level, target_limbs=4, value_target_limbs=3, crypto_context=ctx)
    assert [h.state.cur_limbs for h in dropped.handles] == [4, 4, 3, 3]
    assert all(h.releases == 1 for h in hs) and dropped.column == 4
    with pytest.raises(ValueError, match="needs a refresh to reach"):
        drop_pairfold_token_to_limbs(dropped, target_limbs=5, crypto_context=ctx)
    assert not dropped.is_consumed
    with pytest.raises(ValueError):
        drop_pairfold_token_to_limbs(dropped, target_limbs=1, crypto_context=ctx)
