"""The walk of numpy's pairwise float32 summation that the GlobalAvgPool2d
kernels follow (novann_amd/csrc/novaq_gap_plan.h: the tree made complete, a
virtual leaf per 2^D slot, idle slots holding -0.0f, neighbours added level by
level), for every block size up to 8192: the owned leaves are numpy's leaves
in order, each once; the neighbour-first combination of the virtual leaves is
numpy's recursion, node for node; the depth and leaf lengths the launchers
size the kernels by are right; and evaluated in float32 (blocks of 8192 added
in order from 0, as numpy's reduction does) the walk gives np.mean bit for
bit.  CPU only (the header is built with g++)."""
from __future__ import annotations

import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
f32 = np.float32


def numpy_tree(n, off=0):
    """numpy's pairwise recursion as a nested tuple of (off, len) leaves."""
    if n <= 128:
        return (off, n)
    n2 = n // 2
    n2 -= n2 % 8
    return (numpy_tree(n2, off), numpy_tree(n - n2, off + n2))


def leaves_of(t):
    return [t] if isinstance(t[0], int) else leaves_of(t[0]) + leaves_of(t[1])


def depth_of(t):
    return 0 if isinstance(t[0], int) else 1 + max(depth_of(t[0]), depth_of(t[1]))


def virtual_tree(owners, lo, hi):
    """The neighbour-first combination over virtual leaves [lo, hi): idle
    leaves are the identity, so a range with one owner is that leaf."""
    inside = [v for v in owners if lo <= v < hi]
    if not inside:
        return None
    if len(inside) == 1 and inside[0] == lo:
        return owners[lo]
    mid = (lo + hi) // 2
    left, right = virtual_tree(owners, lo, mid), virtual_tree(owners, mid, hi)
    if left is None or right is None:
        return left if right is None else right
    return (left, right)


@pytest.fixture(scope="module")
def walks(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("gap") / "gap_plan_dump")
    subprocess.run([gxx, "-std=c++17", "-O1", "-Wall", "-o", exe,
                    os.path.join(HERE, "native", "gap_plan_dump.cpp")], check=True)
    out = subprocess.run([exe, "8192"], check=True, capture_output=True, text=True).stdout
    res = {}
    for line in out.splitlines():
        f = line.split()
        n, D, longest, shortest = map(int, f[:4])
        owners = {}
        for item in f[4:]:
            vi, off, ln = map(int, item.split(","))
            owners[vi] = (off, ln)
        res[n] = (D, longest, shortest, owners)
    return res


def test_walk_is_numpys_recursion_for_every_block_size(walks):
    assert len(walks) == 8192
    for n in range(1, 8193):
        D, longest, shortest, owners = walks[n]
        want = numpy_tree(n)
        assert D == depth_of(want), n
        assert all(v < (1 << D) for v in owners), n  # nothing past the tree
        lv = leaves_of(want)
        assert [owners[v] for v in sorted(owners)] == lv, n
        assert longest == max(ln for _, ln in lv) and shortest == min(ln for _, ln in lv), n
        assert virtual_tree(owners, 0, 1 << D) == want, n


def test_the_trees_the_launchers_rely_on(walks):
    # 28 x 28: 8 leaves of 96 / 104 at depth 3 (one virtual leaf each); the
    # deepest trees up to 8192 are 7 levels deep; a leaf never exceeds 128
    assert walks[784][0] == 3 and sorted(walks[784][3]) == list(range(8))
    assert max(w[0] for w in walks.values()) == 7
    assert max(w[1] for w in walks.values()) == 128
    # 250: leaves at unequal depths, virtual leaf 1 idle
    assert walks[250][0] == 2 and sorted(walks[250][3]) == [0, 2, 3]


def _leaf_sum(a):
    """numpy's pairwise leaf in float32: 8 interleaved partial sums, combined
    ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the remainder in order; below 8
    elements a plain sum from 0."""
    n = a.size
    if n < 8:
        s = f32(0.0)
        for v in a:
            s = f32(s + v)
        return s
    main = n - n % 8
    r = a[:8].copy()
    for i in range(8, main, 8):
        r = (r + a[i:i + 8]).astype(np.float32)
    s = f32(f32(f32(r[0] + r[1]) + f32(r[2] + r[3])) + f32(f32(r[4] + r[5]) + f32(r[6] + r[7])))
    for v in a[main:]:
        s = f32(s + v)
    return s


def _walk_sum(walks, a):
    """One block through the walk: leaf sums at their virtual leaves, -0.0 at
    the idle ones, neighbours added level by level."""
    D, _, _, owners = walks[a.size]
    v = [f32(-0.0)] * (1 << D)
    for vi, (off, ln) in owners.items():
        v[vi] = _leaf_sum(a[off:off + ln])
    while len(v) > 1:
        v = [f32(v[i] + v[i + 1]) for i in range(0, len(v), 2)]
    return v[0]


@pytest.mark.parametrize("n", [1, 5, 8, 100, 128, 129, 250, 1000, 4097, 7688, 7689, 7921, 8100,
                               8191, 8192, 8193, 12544, 20000])
def test_walk_evaluates_to_np_mean(walks, n):
    rng = np.random.default_rng(n)
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-6, 6, n))).astype(np.float32)
    total = f32(0.0)
    for b in range(0, n, 8192):  # numpy's blocks, added in order from 0
        total = f32(total + _walk_sum(walks, a[b:b + 8192]))
    got = f32(total / f32(n))
    want = np.mean(a.reshape(1, 1, 1, n), axis=(2, 3), keepdims=True).reshape(())
    assert got.view(np.uint32) == np.float32(want).view(np.uint32)


def test_all_negative_zero_plane_gives_positive_zero(walks):
    a = np.full(784, -0.0, np.float32)
    got = f32(f32(f32(0.0) + _walk_sum(walks, a)) / f32(784))
    assert got.view(np.uint32) == 0
