"""Host logic of HipBackend's plan cache (no GPU): the page-list diff that
becomes dh_plan_update events, and the BlockTable identity / version the
cache is keyed on."""
import numpy as np

from dendrite_amd import _lib
from dendrite_amd.backend import _list_events
from dendrite_amd.cache import BlockTable

A, R = _lib.PLAN_APPEND, _lib.PLAN_REPLACE_LAST


def _ev(old, new):
    return _list_events(np.array(old, np.uint32), np.array(new, np.uint32))


def test_equal_lists_need_no_event():
    assert _ev([], []) == []
    assert _ev([3, 4, 5], [3, 4, 5]) == []


def test_appends():
    assert _ev([3, 4], [3, 4, 9]) == [(A, 9)]
    assert _ev([3, 4], [3, 4, 9, 11]) == [(A, 9), (A, 11)]
    assert _ev([], [7]) == [(A, 7)]          # dh_plan_update refuses it: a new plan follows


def test_replaced_last_page_then_appends():
    assert _ev([3, 4, 5], [3, 4, 8]) == [(R, 8)]
    assert _ev([3, 4, 5], [3, 4, 8, 9]) == [(R, 8), (A, 9)]
    assert _ev([5], [8]) == [(R, 8)]


def test_other_changes_take_a_new_plan():
    assert _ev([3, 4, 5], [3, 4]) is None           # shrank
    assert _ev([3, 4, 5], [3, 9, 5]) is None        # a middle page changed
    assert _ev([3, 4, 5], [6, 4, 5, 7]) is None
    assert _ev([3, 4, 5], []) is None


def test_block_table_version_and_uid():
    t = BlockTable.from_blocks([1, 2])
    u = BlockTable.from_blocks([1, 2])
    assert t.uid != u.uid
    v = t.version
    t.add_tokens(3)                       # token count only: same page list
    assert t.version == v
    t.push(5)
    assert t.version == v + 1
    t.set(0, 9)
    assert t.version == v + 2
    assert list(t.block_ids()) == [9, 2, 5] and t.block_ids().dtype == np.uint32
    f = t.fork()
    assert f.uid not in (t.uid, u.uid) and list(f.block_ids()) == [9, 2, 5]
    t.clear()
    assert t.version == v + 3 and len(t.block_ids()) == 0
