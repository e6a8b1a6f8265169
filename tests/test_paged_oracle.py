"""Pins of the paged-attention oracle (oracle.floatops.paged_attention).

The reference holds no golden vectors for this operator (its tests compute a
host reference, tests/cuda/test_paged_attention.cu:45-103), so the oracle is
pinned by what fixes attention independently of it: torch's
scaled_dot_product_attention on the gathered (contiguous) K and V, closed forms
(a single token returns its V row; identical keys average the values), the
invariances the reference tests (reordering whole blocks of the context leaves
the result unchanged, repointing a table entry at other data changes it), GQA
as repeated KV heads, and planted mistakes that these checks must catch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

from .paged_util import REFERENCE_CASES, make_case


def gathered(case):
    """Contiguous [S, n, KVH, D] K and V of each sequence, by the table."""
    bs = case.k_cache.shape[1]
    out = []
    for s, n in enumerate(case.context):
        t = np.arange(int(n))
        blocks = case.tables[s].astype(np.int64)[t // bs]
        out.append((case.k_cache[blocks, t % bs], case.v_cache[blocks, t % bs]))
    return out


def sdpa(case) -> np.ndarray:
    s_count, heads, dim = case.query.shape
    group = heads // case.k_cache.shape[2]
    out = np.zeros((s_count, heads, dim))
    for s, (k, v) in enumerate(gathered(case)):
        if len(k) == 0:
            continue
        q = torch.from_numpy(case.query[s].astype(np.float64))[:, None, :]          # [H, 1, D]
        kk = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2).repeat_interleave(group, 0)
        vv = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2).repeat_interleave(group, 0)
        o = torch.nn.functional.scaled_dot_product_attention(q, kk.contiguous(), vv.contiguous(),
                                                             scale=case.scale)
        out[s] = o[:, 0, :].numpy()
    return out


def run(case):
    return oracle.paged_attention(case.query, case.k_cache, case.v_cache, case.tables, case.context,
                                  case.scale)


@pytest.mark.parametrize("dims", REFERENCE_CASES + [(2, 8, 2, 80, 16, [40, 0])], ids=str)
def test_oracle_matches_torch_sdpa_on_the_gathered_cache(dims):
    case = make_case(*dims, seed=sum(dims[:5]))
    np.testing.assert_allclose(run(case), sdpa(case), rtol=1e-12, atol=1e-12)


def test_closed_forms():
    case = make_case(1, 2, 1, 32, 4, [1], seed=3)
    block = case.tables[0, 0]
    np.testing.assert_allclose(run(case)[0], np.repeat(case.v_cache[block, 0], 2, 0).reshape(2, 32)
                               .astype(np.float64), rtol=0, atol=0)
    same = make_case(1, 1, 1, 16, 4, [10], seed=4)
    same.k_cache[:] = same.k_cache[0, 0]
    t = np.arange(10)
    rows = same.v_cache[same.tables[0].astype(np.int64)[t // 4], t % 4, 0]
    np.testing.assert_allclose(run(same)[0, 0], rows.astype(np.float64).mean(0), rtol=1e-12, atol=1e-12)
    empty = make_case(2, 2, 2, 16, 4, [0, 6], seed=5)
    assert np.all(run(empty)[0] == 0.0)


def test_invariance_and_table_following():
    case = make_case(1, 1, 1, 32, 4, [8], seed=3)
    base = run(case)
    swapped = make_case(1, 1, 1, 32, 4, [8], seed=3)
    swapped.tables[0, [0, 1]] = swapped.tables[0, [1, 0]]
    np.testing.assert_allclose(run(swapped), base, rtol=1e-12, atol=1e-12)
    repointed = make_case(1, 1, 1, 32, 4, [8], seed=3)
    used = set(repointed.tables[0].tolist())
    repointed.tables[0, 0] = next(b for b in range(repointed.k_cache.shape[0]) if b not in used)
    assert np.abs(run(repointed) - base).max() > 1e-3


def test_gqa_equals_repeated_kv_heads():
    case = make_case(2, 8, 2, 64, 8, [20, 9], seed=5)
    wide = make_case(2, 8, 2, 64, 8, [20, 9], seed=5)
    wide.k_cache = np.repeat(case.k_cache, 4, axis=2)
    wide.v_cache = np.repeat(case.v_cache, 4, axis=2)
    np.testing.assert_allclose(run(case), run(wide), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("mistake", ["ignore_table", "gqa_modulo", "no_scale"])
def test_planted_mistakes_are_caught(mistake):
    case = make_case(2, 4, 2, 32, 4, [9, 6], seed=7)
    expected = sdpa(case)
    wrong = make_case(2, 4, 2, 32, 4, [9, 6], seed=7)
    if mistake == "ignore_table":
        wrong.tables = np.arange(wrong.tables.size, dtype=np.uint32).reshape(wrong.tables.shape)
        got = run(wrong)
    elif mistake == "gqa_modulo":
        # head h reading KV head h % KVH instead of h // (H / KVH)
        perm = [h % 2 * 2 + h // 2 for h in range(4)]
        wrong.query = case.query[:, perm, :]
        got = run(wrong)[:, np.argsort(perm), :]
    else:
        got = oracle.paged_attention(case.query, case.k_cache, case.v_cache, case.tables, case.context, 1.0)
    assert np.abs(got - expected).max() > 1e-3
