"""CPU: the product library's token-tree API against cogito's own compiled
sources (oracle/_ref), src/inference/speculative.c:14-30,184-238.

These entry points are host code in the product library, so they run
without a device.  The drop-in keeps the reference's semantics exactly: the
mask is the chain mask whatever branch_points holds, add_token does nothing,
and free leaves branch_points to its owner.  The tree form of the mask is
the extension cgx_tree_attention_mask_parents, checked against the closed
form (node i sees the prefix, itself and its ancestors).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import CgTokenTree
from oracle_lib import ref_tensor_np

PTREE = C.POINTER(CgTokenTree)


def _np(t, lib_free):
    n = t.contents.size
    shape = tuple(t.contents.shape[i] for i in range(t.contents.ndim))
    out = np.ctypeslib.as_array(t.contents.data, shape=(n,)).copy().reshape(shape)
    lib_free(t)
    return out


def _ref_mask(ref, seqlen, depth):
    tree = ref.cg_token_tree_new(depth)
    m = ref.cg_tree_attention_mask(tree, seqlen)
    got = ref_tensor_np(m)
    ref.cg_tensor_free(m)
    ref.cg_token_tree_free(tree)
    return got


@pytest.mark.parametrize("seqlen,depth", [(0, 1), (7, 4), (1, 9), (33, 6)])
def test_chain_mask_matches_reference(lib, ref, seqlen, depth):
    tree = lib.cg_token_tree_new(depth)
    # a "tree" in branch_points must not change the drop-in mask
    bp = np.array([-1] + [0] * (depth - 1), np.int32)
    tree.contents.branch_points = bp.ctypes.data_as(C.POINTER(C.c_int))
    tree.contents.num_branches = depth
    got = _np(lib.cg_tree_attention_mask(tree, seqlen), lib.cg_tensor_free)
    np.testing.assert_array_equal(got, _ref_mask(ref, seqlen, depth))
    # free leaves branch_points alone (a numpy buffer: freeing it would abort)
    tree.contents.branch_points = None
    lib.cg_token_tree_free(tree)


def test_tree_container_matches_reference(lib, ref):
    depth = 5
    tree = lib.cg_token_tree_new(depth)
    rtree = C.cast(ref.cg_token_tree_new(depth), PTREE)
    for t in (tree, rtree):
        assert t.contents.depth == depth and not t.contents.draft_probs
        for i in range(depth):
            t.contents.tokens[i] = 100 + 7 * i
            assert t.contents.accepted[i] is False
    # add_token is the reference's no-op
    probs = np.ones(4, np.float32)
    lib.cg_token_tree_add_token(tree, 3, probs.ctypes.data_as(C.POINTER(C.c_float)))
    assert tree.contents.depth == depth and tree.contents.tokens[depth - 1] == 128
    got = _np(lib.cg_token_tree_to_tensor(tree), lib.cg_tensor_free)
    rt = ref.cg_token_tree_to_tensor(C.cast(rtree, C.c_void_p))
    exp = ref_tensor_np(rt)
    ref.cg_tensor_free(rt)
    np.testing.assert_array_equal(got, exp)
    # free with a caller-owned branch_points buffer
    bp = np.zeros(depth, np.int32)
    tree.contents.branch_points = bp.ctypes.data_as(C.POINTER(C.c_int))
    lib.cg_token_tree_free(tree)
    ref.cg_token_tree_free(C.cast(rtree, C.c_void_p))


def _closed_form(parents, seqlen):
    n = len(parents)
    S = seqlen + n
    m = np.full((S, S), -1e9, np.float32)
    for i in range(seqlen):
        m[i, :i + 1] = 0
    for i in range(n):
        m[seqlen + i, :seqlen] = 0
        a = i
        while a >= 0:
            m[seqlen + i, seqlen + a] = 0
            a = parents[a]
    return m


@pytest.mark.parametrize("parents,seqlen", [
    ([-1, 0, 0, 1, 1, 2, 3], 5),
    ([-1, -1, 0, 1], 0),                   # two roots
    ([-1, 0, 1, 2, 3, 4], 9),               # a chain
])
def test_parents_mask_closed_form(lib, ref, parents, seqlen):
    p = np.array(parents, np.int32)
    t = lib.cgx_tree_attention_mask_parents(p.ctypes.data, len(p), seqlen)
    got = _np(t, lib.cg_tensor_free).reshape(seqlen + len(p), -1)
    np.testing.assert_array_equal(got, _closed_form(parents, seqlen))
    if parents == list(range(-1, len(parents) - 1)):
        S = seqlen + len(p)
        np.testing.assert_array_equal(got, _ref_mask(ref, seqlen, len(p)).reshape(S, S))


def test_parents_mask_rejects_bad_parents(lib):
    p = np.array([-1, 1], np.int32)
    assert not lib.cgx_tree_attention_mask_parents(p.ctypes.data, 2, 3)
    lib.cgx_clear_error()
