"""The host plan of numpy's pairwise float32 summation that the GlobalAvgPool2d
wave kernel follows (novann_amd/csrc/novaq_gap_plan.h), for every plane size
up to 8192 and beyond: its leaves and postfix program against a restatement
of numpy's split (n2 = n/2 - (n/2) % 8, leaves of <= 128 elements), its
capacity (65 leaves for every n in [7689, 8191]), and numerically: evaluating
a plane through the plan in float32 gives np.mean bit for bit.  CPU only (the
helper is built with g++)."""
from __future__ import annotations

import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def numpy_split(n, off=0, leaves=None, prog=None):
    """numpy's pairwise recursion: (leaves as (off, len), postfix ops)."""
    if leaves is None:
        leaves, prog = [], []
    if n <= 128:
        leaves.append((off, n))
        prog.append(1)
        return leaves, prog
    n2 = n // 2
    n2 -= n2 % 8
    numpy_split(n2, off, leaves, prog)
    numpy_split(n - n2, off + n2, leaves, prog)
    prog.append(0)
    return leaves, prog


@pytest.fixture(scope="module")
def plans(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("gap") / "gap_plan_dump")
    subprocess.run([gxx, "-std=c++17", "-O1", "-Wall", "-o", exe,
                    os.path.join(HERE, "native", "gap_plan_dump.cpp")], check=True)
    out = subprocess.run([exe, "9000"], check=True, capture_output=True, text=True).stdout
    res = {}
    for line in out.splitlines():
        f = line.split()
        n, ok, L, nops, bal = map(int, f[:5])
        if not ok:
            res[n] = None
            continue
        words = len(f) - 5 - L
        prog_words = [int(v) for v in f[5:5 + words]]
        leaves = [tuple(map(int, v.split(","))) for v in f[5 + words:]]
        prog = [(prog_words[k >> 5] >> (k & 31)) & 1 for k in range(nops)]
        res[n] = (L, nops, leaves, prog, bal)
    return res


def test_plan_matches_numpy_split_for_every_plane_size(plans):
    assert len(plans) == 9000
    for n in range(1, 8193):
        assert plans[n] is not None, n
        L, nops, leaves, prog = plans[n][:4]
        want_leaves, want_prog = numpy_split(n)
        assert leaves == want_leaves and prog == want_prog, n
        assert L == len(leaves) and nops == 2 * L - 1, n


def complete_tree_prog(L):
    """Postfix program of the complete binary tree over L = 2^d leaves."""
    if L == 1:
        return [1]
    half = complete_tree_prog(L // 2)
    return half + half + [0]


def test_balanced_flag_marks_exactly_the_complete_trees(plans):
    # the kernel adds such plans' leaf sums by pairwise shuffles (neighbours,
    # then pairs of pairs): that is the program's association exactly when the
    # program is the complete tree's; plane sizes up to 1024 (32 x 32) cover
    # every L in {1, 2, 4, 8}
    seen = set()
    for n in range(1, 8193):
        L, nops, leaves, prog, bal = plans[n]
        complete = L in (1, 2, 4, 8) and prog == complete_tree_prog(L)
        assert bool(bal) == complete, n
        if bal:
            seen.add(L)
    assert seen == {1, 2, 4, 8}
    assert plans[784][4] == 1 and plans[49][4] == 1 and plans[196][4] == 1
    assert plans[7921][4] == 0


def test_capacity_covers_65_leaves():
    # the bound the plan has to hold: 441 sizes below 8192 need 65 leaves
    big = [n for n in range(1, 8193) if len(numpy_split(n)[0]) > 64]
    assert len(big) == 441 and big[0] == 7689 and big[-1] == 8191
    assert max(len(numpy_split(n)[0]) for n in range(1, 8193)) == 65


def test_plan_stack_depth_fits(plans):
    for n in range(1, 8193):
        depth = best = 0
        for op in plans[n][3]:
            depth = depth + 1 if op else depth - 1
            best = max(best, depth)
        assert best <= 8, n  # the kernel's register stack


def _leaf_sum(a):
    """numpy's pairwise leaf in float32: 8 interleaved partial sums, combined
    ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the remainder in order; below 8
    elements a plain sum from 0."""
    n = a.size
    if n < 8:
        s = np.float32(0.0)
        for v in a:
            s = np.float32(s + v)
        return s
    main = n - n % 8
    r = a[:8].copy()
    for i in range(8, main, 8):
        r = (r + a[i:i + 8]).astype(np.float32)
    f = np.float32
    s = f(f(f(r[0] + r[1]) + f(r[2] + r[3])) + f(f(r[4] + r[5]) + f(r[6] + r[7])))
    for v in a[main:]:
        s = f(s + v)
    return s


@pytest.mark.parametrize("n", [1, 5, 8, 100, 128, 129, 1000, 4097, 7688, 7689, 7921, 8100,
                               8191, 8192])
def test_plan_evaluates_to_np_mean(plans, n):
    rng = np.random.default_rng(n)
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-6, 6, n))).astype(np.float32)
    L, nops, leaves, prog = plans[n][:4]
    sums = [_leaf_sum(a[o:o + ln]) for o, ln in leaves]
    st, k = [], 0
    for op in prog:
        if op:
            st.append(sums[k])
            k += 1
        else:
            b2 = st.pop()
            st.append(np.float32(st.pop() + b2))
    got = np.float32(np.float32(0.0) + st[0]) / np.float32(n)
    want = np.mean(a.reshape(1, 1, 1, n), axis=(2, 3), keepdims=True).reshape(())
    assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32)


def test_plan_refuses_what_it_cannot_hold(plans):
    # above one numpy buffer block the kernel never plans; sizes whose tree
    # would overflow the capacity are refused rather than written past it
    for n in range(8193, 9001):
        p = plans[n]
        if p is not None:
            assert p[0] <= 80 and p[1] == 2 * p[0] - 1
