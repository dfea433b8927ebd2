"""GPU: cogito's speculative-decoding driver API (include/cg_speculative.h:71-130,
declared only in the reference) through the C ABI.

* cg_target_verify on given logits: the accept / reject decisions, the
  correction or bonus token, accepted[], the decoder statistics and the
  global LCG's state equal the oracle's chain verify (orc_verify_chain) fed
  by a mirror of the reference's LCG (src/inference/speculative.c:11-12).
* cg_speculative_step / cg_draft_generate on two synthetic models: draft and
  target logits within 1e-3 of the oracle stack (tests/oracle_model.py);
  every drafted token is the oracle sampler's draw from those logits with
  the mirrored LCG, and the verify decisions are the oracle's, bit for bit.
* cg_speculative_generate equals the same steps made one by one, and a draft
  identical to the target accepts every drafted token.
* cg_forward_tree_attention: rows of the causal prefix and of a tree under
  cgx_tree_attention_mask_parents match the oracle stack run over the
  prefix plus each node's ancestor path.
* cg_eagle_generate_tree: the draft's most likely token at each depth;
  cg_eagle_compute_branching: the number of top tokens reaching 0.8 of the
  draft's softmax mass (decision D17).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cogito_amd.capi import last_error
from gpu_util import host_tensor, rel_err_rows, tensor_np
from oracle_lib import LCG, ptr
from oracle_model import Cfg, OracleModel

pytestmark = pytest.mark.gpu
TOL = 1e-3

TARGET = Cfg(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512,
             vocab=1024, group_size=128, kv_group_size=64, max_seq=96, max_tokens=8,
             init_std=0.05)
DRAFT = Cfg(**{**TARGET.__dict__, "n_layers": 1})


def new_model(gpu, cfg, seed):
    cc = cfg.ctype()
    m = gpu.cgx_model_new(C.byref(cc), seed, None)
    assert m, last_error(gpu)
    return m


def ids_tensor(gpu, ids):
    return host_tensor(gpu, np.asarray(ids, np.float32).reshape(1, -1))


def rows(ptr_f, n):
    return np.ctypeslib.as_array(ptr_f, shape=(n,)).copy()


def filtered_draw(oracle, row, T, k, p, u):
    r = np.ascontiguousarray(row, np.float32)
    return oracle.orc_sample_filtered(ptr(r), r.size, T, k, p, u)


def oracle_verify(oracle, tl, dl, tok, u, g, V, T, k, p):
    out = np.zeros(g + 1, np.int32)
    n = oracle.orc_verify_chain(ptr(np.ascontiguousarray(tl, np.float32)),
                                ptr(np.ascontiguousarray(dl, np.float32)),
                                ptr(np.ascontiguousarray(tok, np.int32)),
                                ptr(np.asarray(u, np.float32)), g, V, T, k, p, ptr(out), None)
    return n, out


FILTERS = [(1.0, 0, 1.0), (0.8, 0, 0.9), (0.7, 50, 0.9), (1.0, 20, 1.0)]


@pytest.mark.parametrize("T,top_k,top_p", FILTERS)
def test_target_verify_given_logits(gpu, oracle, rng, T, top_k, top_p):
    V, g = TARGET.vocab, 4
    tm = new_model(gpu, TARGET, 3)
    dec = gpu.cg_speculative_decoder_new(None, tm, g)
    dec.contents.temperature, dec.contents.top_k, dec.contents.top_p = T, top_k, top_p
    tree = gpu.cg_token_tree_new(g)
    seen = set()
    for trial in range(12):
        tl = rng.normal(0, 2, (g + 1, V)).astype(np.float32)
        dl = (tl[:g] + rng.normal(0, 0.7, (g, V))).astype(np.float32)
        state = int(rng.integers(0, 2**32))
        mirror = LCG(state)
        pre = [mirror.draw(oracle) for _ in range(g + 1)]
        # drafts: the filtered draft distribution's likely tokens, sometimes not
        tok = np.array([int(np.argmax(dl[i])) if rng.random() < 0.7 else
                        int(rng.integers(0, V)) for i in range(g)], np.int32)
        n_exp, out_exp = oracle_verify(oracle, tl, dl, tok, pre, g, V, T, top_k, top_p)
        seen.add(n_exp)
        for i in range(g):
            tree.contents.tokens[i] = int(tok[i])
        tree.contents.draft_probs = dl.ctypes.data_as(C.POINTER(C.c_float))
        tree.contents.target_probs = tl.ctypes.data_as(C.POINTER(C.c_float))
        gpu.cgx_lcg_seed(state)
        before = (dec.contents.total_draft_tokens, dec.contents.accepted_draft_tokens,
                  dec.contents.num_steps)
        n = gpu.cg_target_verify(dec, None, tree)
        assert n == n_exp, (trial, n, n_exp, last_error(gpu))
        assert [tree.contents.accepted[i] for i in range(g)] == [i < n for i in range(g)]
        if n < g:
            assert tree.contents.tokens[n] == out_exp[n]
        assert gpu.cgx_last_verify_token() == out_exp[n]
        # the LCG advanced by the draws a sequential verify makes
        used = n + 2 if n < g else g + 1
        lcg = LCG(state)
        for _ in range(used):
            lcg.draw(oracle)
        assert gpu.cgx_lcg_state() == lcg.state.value
        assert (dec.contents.total_draft_tokens, dec.contents.accepted_draft_tokens,
                dec.contents.num_steps) == (before[0] + g, before[1] + n, before[2] + 1)
        assert dec.contents.avg_acceptance_rate == pytest.approx(
            dec.contents.accepted_draft_tokens / dec.contents.total_draft_tokens, rel=1e-6)
    assert len(seen) >= 2, seen
    tree.contents.draft_probs = None
    tree.contents.target_probs = None
    gpu.cg_token_tree_free(tree)
    gpu.cg_speculative_decoder_free(dec)
    gpu.cgx_model_free(tm)


def _check_step(gpu, oracle, dec, tree, prompt, n_acc, state, T, k, p, g):
    """Draft and target logits against the oracle stacks, drafted tokens and
    verify decisions against the oracle's draws (mirrored LCG)."""
    V = TARGET.vocab
    dl = rows(tree.contents.draft_probs, g * V).reshape(g, V)
    tl = rows(tree.contents.target_probs, (g + 1) * V).reshape(g + 1, V)
    tok = np.array([tree.contents.tokens[i] for i in range(g)], np.int32)
    lcg = LCG(state)
    ud = [lcg.draw(oracle) for _ in range(g)]
    uv = [lcg.draw(oracle) for _ in range(g + 1)]
    drafted = []
    for i in range(g):
        drafted.append(filtered_draw(oracle, dl[i], T, k, p, ud[i]))
    # the drafted tokens, except the one the correction overwrote
    for i in range(g):
        if not (i == n_acc and n_acc < g):
            assert tok[i] == drafted[i], (i, tok[i], drafted[i])
    n_exp, out = oracle_verify(oracle, tl, dl, np.array(drafted, np.int32), uv, g, V, T, k, p)
    assert n_acc == n_exp
    assert gpu.cgx_last_verify_token() == out[n_acc]
    if n_acc < g:
        assert tok[n_acc] == out[n_acc]
    # logits against the oracle stacks over prompt + drafts
    seq = list(prompt) + drafted
    od = OracleModel(oracle, DRAFT, 21)
    od_rows = od.forward(seq[:len(prompt) + g - 1], g)
    assert rel_err_rows(dl, od_rows) < TOL
    ot = OracleModel(oracle, TARGET, 20)
    ot_rows = ot.forward(seq[:len(prompt) + g], g + 1)
    assert rel_err_rows(tl, ot_rows) < TOL
    return [int(t) for t in out[:n_acc + 1]]


@pytest.mark.parametrize("T,top_k,top_p", FILTERS[:3])
def test_speculative_step_vs_oracle(gpu, oracle, rng, T, top_k, top_p):
    g = 3
    tm = new_model(gpu, TARGET, 20)
    dm = new_model(gpu, DRAFT, 21)
    dec = gpu.cg_speculative_decoder_new(dm, tm, g)
    dec.contents.temperature, dec.contents.top_k, dec.contents.top_p = T, top_k, top_p
    prompt = [int(x) for x in rng.integers(0, TARGET.vocab, 11)]
    tree = gpu.cg_token_tree_new(g)
    for step in range(3):
        state = int(rng.integers(0, 2**32))
        gpu.cgx_lcg_seed(state)
        ids = ids_tensor(gpu, prompt)
        n = gpu.cg_speculative_step(dec, ids, tree)
        gpu.cg_tensor_free(ids)
        assert 0 <= n <= g, last_error(gpu)
        emitted = _check_step(gpu, oracle, dec, tree, prompt, n, state, T, top_k, top_p, g)
        # the target keeps the last input token and the accepted drafts
        assert gpu.cgx_model_len(tm) == len(prompt) + n
        prompt += emitted
    assert dec.contents.num_steps == 3 and dec.contents.total_draft_tokens == 3 * g
    gpu.cg_token_tree_free(tree)
    gpu.cg_speculative_decoder_free(dec)
    gpu.cgx_model_free(dm)
    gpu.cgx_model_free(tm)


def test_draft_generate_vs_oracle(gpu, oracle, rng):
    g, T = 4, 0.9
    dm = new_model(gpu, DRAFT, 21)
    dec = gpu.cg_speculative_decoder_new(dm, None, g)
    dec.contents.temperature, dec.contents.top_k, dec.contents.top_p = T, 0, 1.0
    prompt = [int(x) for x in rng.integers(0, TARGET.vocab, 9)]
    state = 777
    gpu.cgx_lcg_seed(state)
    ids = ids_tensor(gpu, prompt)
    tree = gpu.cg_draft_generate(dec, ids)
    assert tree, last_error(gpu)
    V = TARGET.vocab
    dl = rows(tree.contents.draft_probs, g * V).reshape(g, V)
    lcg = LCG(state)
    tok = [filtered_draw(oracle, dl[i], T, 0, 1.0, lcg.draw(oracle)) for i in range(g)]
    assert [tree.contents.tokens[i] for i in range(g)] == tok
    assert gpu.cgx_lcg_state() == lcg.state.value
    od = OracleModel(oracle, DRAFT, 21)
    assert rel_err_rows(dl, od.forward(prompt + tok[:g - 1], g)) < TOL
    gpu.cg_token_tree_free(tree)
    gpu.cg_tensor_free(ids)
    gpu.cg_speculative_decoder_free(dec)
    gpu.cgx_model_free(dm)


def test_generate_equals_steps_and_identical_draft_accepts_all(gpu, rng):
    g, T, top_p = 3, 0.8, 0.95
    tm = new_model(gpu, TARGET, 20)
    dm = new_model(gpu, DRAFT, 21)
    prompt = [int(x) for x in rng.integers(0, TARGET.vocab, 7)]
    dec = gpu.cg_speculative_decoder_new(dm, tm, g)
    ids = ids_tensor(gpu, prompt)
    gpu.cgx_lcg_seed(99)
    res = gpu.cg_speculative_generate(dec, ids, 20, T, top_p)
    assert res, last_error(gpu)
    gen = tensor_np(gpu, res).ravel().astype(int).tolist()
    assert gen[:len(prompt)] == prompt and len(gen) == len(prompt) + 20
    gpu.cg_tensor_free(res)
    # the same steps one by one (same decoder settings, same LCG start)
    dec2 = gpu.cg_speculative_decoder_new(dm, tm, g)
    dec2.contents.temperature, dec2.contents.top_p = T, top_p
    gpu.cgx_lcg_seed(99)
    seq = list(prompt)
    tree = gpu.cg_token_tree_new(g)
    while len(seq) < len(gen):
        t = ids_tensor(gpu, seq)
        n = gpu.cg_speculative_step(dec2, t, tree)
        gpu.cg_tensor_free(t)
        assert n >= 0, last_error(gpu)
        seq += [tree.contents.tokens[i] for i in range(n)] + [gpu.cgx_last_verify_token()]
    assert seq[:len(gen)] == gen
    assert dec.contents.num_steps == dec2.contents.num_steps
    gpu.cg_token_tree_free(tree)
    gpu.cg_speculative_decoder_free(dec2)
    gpu.cg_speculative_decoder_free(dec)
    # a draft with the target's weights (separate caches) accepts everything
    twin = new_model(gpu, TARGET, 20)
    dec3 = gpu.cg_speculative_decoder_new(twin, tm, g)
    gpu.cgx_lcg_seed(5)
    res = gpu.cg_speculative_generate(dec3, ids, 16, 1.0, 1.0)
    assert res, last_error(gpu)
    assert dec3.contents.accepted_draft_tokens == dec3.contents.total_draft_tokens > 0
    gpu.cg_tensor_free(res)
    gpu.cg_tensor_free(ids)
    gpu.cg_speculative_decoder_free(dec3)
    for m in (twin, dm, tm):
        gpu.cgx_model_free(m)


def test_forward_tree_attention_vs_oracle(gpu, oracle, rng):
    V = TARGET.vocab
    m = new_model(gpu, TARGET, 20)
    prompt = [int(x) for x in rng.integers(0, V, 10)]
    parents = [-1, 0, 0, 1, 1, 2]
    nodes = [int(x) for x in rng.integers(0, V, len(parents))]
    p = np.array(parents, np.int32)
    mask = gpu.cgx_tree_attention_mask_parents(p.ctypes.data, len(p), len(prompt))
    assert mask, last_error(gpu)
    ids = ids_tensor(gpu, prompt + nodes)
    out = gpu.cg_forward_tree_attention(m, ids, mask)
    assert out, last_error(gpu)
    got = tensor_np(gpu, out).reshape(len(prompt) + len(nodes), V)
    om = OracleModel(oracle, TARGET, 20)
    assert rel_err_rows(got[:len(prompt)], om.forward(prompt)) < TOL
    for i in range(len(nodes)):
        path, a = [], i
        while a >= 0:
            path.append(nodes[a])
            a = parents[a]
        om = OracleModel(oracle, TARGET, 20)
        ref = om.forward(prompt + path[::-1], 1)
        assert rel_err_rows(got[len(prompt) + i:len(prompt) + i + 1], ref) < TOL, i
    # the reference's chain mask: a causal forward of every row
    tree = gpu.cg_token_tree_new(len(nodes))
    chain = gpu.cg_tree_attention_mask(tree, len(prompt))
    out2 = gpu.cg_forward_tree_attention(m, ids, chain)
    assert out2, last_error(gpu)
    got2 = tensor_np(gpu, out2).reshape(-1, V)
    om = OracleModel(oracle, TARGET, 20)
    assert rel_err_rows(got2, om.forward(prompt + nodes)) < TOL
    for t in (out, out2, mask, chain, ids):
        gpu.cg_tensor_free(t)
    gpu.cg_token_tree_free(tree)
    gpu.cgx_model_free(m)


def test_eagle_generate_tree(gpu, oracle, rng):
    V, depth = TARGET.vocab, 5
    dm = new_model(gpu, DRAFT, 21)
    e = gpu.cg_eagle_draft_new(dm)
    prompt = [int(x) for x in rng.integers(0, V, 6)]
    ids = ids_tensor(gpu, prompt)
    tree = gpu.cg_eagle_generate_tree(e, ids, depth)
    assert tree, last_error(gpu)
    dl = rows(tree.contents.draft_probs, depth * V).reshape(depth, V)
    tok = [tree.contents.tokens[i] for i in range(depth)]
    assert tok == [int(np.argmax(r)) for r in dl]
    od = OracleModel(oracle, DRAFT, 21)
    assert rel_err_rows(dl, od.forward(prompt + tok[:depth - 1], depth)) < TOL
    gpu.cg_token_tree_free(tree)
    gpu.cg_eagle_draft_free(e)
    # not a model: the reference's placeholder tree
    e2 = gpu.cg_eagle_draft_new(None)
    t2 = gpu.cg_eagle_generate_tree(e2, ids, 3)
    assert [t2.contents.tokens[i] for i in range(3)] == [1, 1, 1]
    gpu.cg_token_tree_free(t2)
    gpu.cg_eagle_draft_free(e2)
    gpu.cg_tensor_free(ids)
    gpu.cgx_model_free(dm)


def test_eagle_compute_branching(gpu, oracle, rng):
    # decision D17: per row, the number of most likely tokens (1..4) whose
    # softmax probabilities first sum to 0.8, against the oracle's softmax
    V = DRAFT.vocab
    x = rng.normal(0, 1, (6, V)).astype(np.float32)
    x[0, 17] = 20.0                              # confident: one branch
    x[1, [3, 4]] = 12.0                          # two equal peaks: two
    x[2] = 0.0                                   # flat: four
    x[3, [5, 6, 7]] = [9.0, 8.5, 8.0]
    exp = []
    for row in x:
        p = np.zeros(V, np.float32)
        oracle.orc_temperature_probs(ptr(np.ascontiguousarray(row)), V, 1.0, ptr(p))
        top = p[np.argsort(-p, kind="stable")[:4]]
        c = np.add.accumulate(top, dtype=np.float32)
        hit = np.flatnonzero(c >= np.float32(0.8))
        exp.append(int(hit[0]) + 1 if hit.size else 4)
    assert exp[:3] == [1, 2, 4]
    dm = new_model(gpu, DRAFT, 21)
    e = gpu.cg_eagle_draft_new(dm)
    t = host_tensor(gpu, x)
    out = gpu.cg_eagle_compute_branching(e, t)
    assert out, last_error(gpu)
    assert [out[i] for i in range(6)] == exp
    C.CDLL(None).free(C.cast(out, C.c_void_p))
    gpu.cg_tensor_free(t)
    gpu.cg_eagle_draft_free(e)
    gpu.cgx_model_free(dm)


@pytest.mark.parametrize("T,top_k,top_p", [(0.8, 0, 0.9), (0.7, 50, 0.9)])
def test_spec_loop_equals_driver_steps(gpu, oracle, rng, T, top_k, top_p):
    """The device loop (cgx_spec_step: each filtered draft draw also writes
    the draft row's filtered distribution, which the verify then uses) and
    the driver (cg_speculative_step: the verify filters the draft logits
    again) on identical model pairs with the same draws emit the same tokens
    at every step.  The driver takes its draws from the global LCG (gamma
    for the drafts, then the verify's, of which it keeps n + 2 on a reject at
    n and gamma + 1 when all are accepted); the loop gets the mirror's."""
    g, seed, steps = 4, 123, 8
    loop_t, loop_d = new_model(gpu, TARGET, 51), new_model(gpu, DRAFT, 52)
    drv_t, drv_d = new_model(gpu, TARGET, 51), new_model(gpu, DRAFT, 52)
    prompt = [int(x) for x in rng.integers(0, TARGET.vocab, 6)]
    s = gpu.cgx_spec_new(loop_d, loop_t, g, T, top_k, top_p)
    assert s, last_error(gpu)
    pr = np.asarray(prompt, np.int32)
    assert gpu.cgx_spec_prefill(s, pr.ctypes.data, len(pr)) == 0, last_error(gpu)
    dec = gpu.cg_speculative_decoder_new(drv_d, drv_t, g)
    dec.contents.temperature, dec.contents.top_k, dec.contents.top_p = T, top_k, top_p
    tree = gpu.cg_token_tree_new(g)
    gpu.cgx_lcg_seed(seed)
    lcg = LCG(seed)
    seq = list(prompt)
    for step in range(steps):
        ids = ids_tensor(gpu, seq)
        n = gpu.cg_speculative_step(dec, ids, tree)
        gpu.cg_tensor_free(ids)
        assert n >= 0, last_error(gpu)
        drv = [tree.contents.tokens[i] for i in range(n)] + [gpu.cgx_last_verify_token()]
        ud = np.array([lcg.draw(oracle) for _ in range(g)], np.float32)
        state_v = lcg.state.value
        uv = np.array([lcg.draw(oracle) for _ in range(g + 1)], np.float32)
        out = np.zeros(g + 1, np.int32)
        m = gpu.cgx_spec_step(s, ud.ctypes.data, uv.ctypes.data, out.ctypes.data)
        assert m == n and out[:n + 1].tolist() == drv, (step, m, out.tolist(), n, drv)
        # the draws the sequential reference consumed
        lcg = LCG(state_v)
        for _ in range(n + 2 if n < g else g + 1):
            lcg.draw(oracle)
        assert gpu.cgx_lcg_state() == lcg.state.value
        seq += drv
    gpu.cg_token_tree_free(tree)
    gpu.cg_speculative_decoder_free(dec)
    gpu.cgx_spec_free(s)
    for m_ in (loop_t, loop_d, drv_t, drv_d):
        gpu.cgx_model_free(m_)
