"""Launch epochs of the one-token kernels, modelled on the CPU through the library's own tag
function (moa_test_epoch_tag runs the code the kernels run; no device is touched).

A one-token QKV, O or FFN launch (and the FFN of 2..16 rows) tags its cross-workgroup hand-off words with a tag that every
workgroup derives from the value its add to a 64-bit epoch counter returned. The model replays
launches in which the workgroups add in arbitrary orders and checks, around every wrap point a
counter or a tag could reach, that (1) all workgroups of a launch derive the same tag, (2) the tag
differs from the previous launch's (a word left by that launch must not pass as current), and
(3) the tag is never 0 (the value of a zero-filled slot). The last test shows that the former
scheme -- 32-bit counters shared by 15 workgroups, tag = old / 15 + 1 -- breaks at the first
counter wrap, since 2^32 mod 15 == 1."""
import ctypes as C
import random

import pytest

from moa_amd import _lib

KERNELS = {0: "qkv", 1: "o", 2: "ffn", 3: "rows ffn"}
GRID = {0: 256, 1: 240, 2: 240, 3: 256}  # workgroups of the one-launch kernels


def layout(kernel):
    n, per = C.c_int(), C.c_int()
    _lib.check(_lib.load().moa_test_epoch_layout(kernel, C.byref(n), C.byref(per)))
    return n.value, per.value


def tag(kernel, old):
    t = C.c_uint32()
    _lib.check(_lib.load().moa_test_epoch_tag(kernel, old, C.byref(t)))
    return t.value


def replay(kernel, start_launches, launches, seed, width=64):
    """Runs `launches` launches from counters preset as after `start_launches` launches (what
    moa_test_preset_epochs does); returns each launch's tag (asserting agreement)."""
    n, per = layout(kernel)
    assert n * per == GRID[kernel] or kernel == 0 and n * per == GRID[0]
    mask = (1 << width) - 1
    counters = [(start_launches * per) & mask] * n
    rng = random.Random(seed)
    tags = []
    for _ in range(launches):
        order = list(range(GRID[kernel]))
        rng.shuffle(order)  # workgroups arrive in any order
        seen = set()
        for b in order:
            c = b % n
            old = counters[c]
            counters[c] = (old + 1) & mask
            seen.add(tag(kernel, old))
        assert len(seen) == 1, f"{KERNELS[kernel]}: workgroups of one launch disagree: {sorted(seen)[:4]}"
        tags.append(seen.pop())
    return tags


WRAPS = [0, 2**28 - 3, 2**29 - 3, 2**32 - 4, 2**32 // 15 - 2, 2**60 // 16 - 3]


@pytest.mark.parametrize("kernel", [0, 1, 2, 3])
@pytest.mark.parametrize("start", WRAPS)
def test_every_launch_agrees_and_differs_from_the_last(kernel, start):
    tags = replay(kernel, start, 7, seed=start ^ kernel)
    assert all(t != 0 for t in tags)
    assert all(a != b for a, b in zip(tags, tags[1:])), tags


def test_tag_is_launch_count_mod_2_32_minus_1_plus_1():
    """Closed form at the tag's own wrap: launch 2^32 - 2 has tag 2^32 - 1, launch 2^32 - 1 wraps to 1."""
    for kernel in KERNELS:
        _, per = layout(kernel)
        assert tag(kernel, 0) == 1
        assert tag(kernel, per - 1) == 1
        assert tag(kernel, per) == 2
        assert tag(kernel, (2**32 - 2) * per) == 2**32 - 1
        assert tag(kernel, (2**32 - 1) * per) == 1
        assert tag(kernel, (2**32) * per) == 2


def test_per_counter_is_a_power_of_two_and_layout_covers_the_grid():
    for kernel in KERNELS:
        n, per = layout(kernel)
        assert per & (per - 1) == 0
        assert n * per == GRID[kernel]


def test_former_scheme_breaks_at_the_32_bit_wrap():
    """The model catches the old bug: 15 workgroups per 32-bit counter, tag = old // 15 + 1."""
    n, per, grid = 16, 15, 240
    counters = [(2**32 - 2 * per) & 0xFFFFFFFF] * n  # two launches before the wrap
    split = False
    for _ in range(4):
        seen = set()
        for b in range(grid):
            old = counters[b % n]
            counters[b % n] = (old + 1) & 0xFFFFFFFF
            seen.add(old // per + 1)
        split |= len(seen) > 1
    assert split


def test_bad_kernel_index_is_rejected():
    lib = _lib.load()
    t = C.c_uint32()
    assert lib.moa_test_epoch_tag(4, 0, C.byref(t)) == -1
    n, per = C.c_int(), C.c_int()
    assert lib.moa_test_epoch_layout(-1, C.byref(n), C.byref(per)) == -1
