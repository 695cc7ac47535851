"""Pin the CPU oracle (oracle/) against things it does not restate.

CPU only.  Each function of oracle/attn_oracle.py is checked against an
independent computation -- a brute-force C triple loop (oracle/cpu_attn.c,
restating tests/test_flash_attn.cu:119-169), torch's CPU
scaled_dot_product_attention in fp64, libstdc++'s own RNG, closed forms,
invariants and the reference's own known-answer smoke test
(kernel_models/flash_attn.py:269-281; the reference ships no fixture files)
-- and planted mistakes in the oracle are shown to fail those checks.
"""
import os
import subprocess
import tempfile

import numpy as np
import pytest

from oracle import attn_oracle as orc
from oracle import c_oracle


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


# ---------------------------------------------------------------------------
# Input generation
# ---------------------------------------------------------------------------
_STD_RNG_SRC = r"""
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
int main(int argc, char** argv) {
    unsigned seed = (unsigned)strtoul(argv[1], 0, 10);
    int n = atoi(argv[2]);
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    for (int i = 0; i < n; ++i) {
        float x = dist(rng);
        unsigned u; std::memcpy(&u, &x, 4);
        std::printf("%08x\n", u);
    }
}
"""


@pytest.fixture(scope="module")
def std_rng_exe():
    d = tempfile.mkdtemp()
    src = os.path.join(d, "rng.cpp")
    exe = os.path.join(d, "rng")
    with open(src, "w") as f:
        f.write(_STD_RNG_SRC)
    subprocess.run(["g++", "-O2", "-o", exe, src], check=True)
    return exe


@pytest.mark.parametrize("seed", [100, 101, 202, 305, 403, 42, 0, 4294967295])
def test_mt19937_uniform_matches_libstdcxx(std_rng_exe, seed):
    n = 4096
    out = subprocess.run([std_rng_exe, str(seed), str(n)], capture_output=True, text=True,
                         check=True).stdout.split()
    expect = np.array([int(x, 16) for x in out], dtype=np.uint32)
    got = orc.mt19937_uniform_f32(n, -1.0, 1.0, seed).view(np.uint32)
    assert np.array_equal(got, expect)


def test_fp16_round_matches_c_rne():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 5.960464477539063e-08, 6.1e-05, 1 + 2.0 ** -11,
                  1 + 3 * 2.0 ** -12, np.inf, -np.inf], dtype=np.float32),
    ])
    ours = orc.fp16_round(vals).view(np.uint16)
    c = np.array([c_oracle.float_to_half_bits(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(ours, c)
    back = np.array([c_oracle.half_bits_to_float(int(h)) for h in c], dtype=np.float32)
    assert np.array_equal(back, ours.view(np.float16).astype(np.float32))


def test_normal_inputs_seed_convention():
    q, k, v = orc.normal_fp16_inputs(1, 4, 2, 3, 5, 16, 7)
    assert q.dtype == np.float16 and q.shape == (1, 4, 3, 16) and k.shape == (1, 2, 5, 16)
    q2 = np.random.default_rng(7).standard_normal((1, 4, 3, 16), dtype=np.float32).astype(np.float16)
    k2 = np.random.default_rng(8).standard_normal((1, 2, 5, 16), dtype=np.float32).astype(np.float16)
    assert np.array_equal(q, q2) and np.array_equal(k, k2)


# ---------------------------------------------------------------------------
# sdpa against the brute-force C restatement and torch
# ---------------------------------------------------------------------------
SHAPES = [
    # B, H_q, H_kv, q_len, kv_len, D
    (1, 1, 1, 16, 16, 16),
    (2, 4, 2, 7, 13, 64),
    (1, 40, 8, 3, 9, 128),   # non-power-of-two GQA ratio (reference case 303)
    (1, 8, 1, 1, 50, 128),   # MQA decode
    (3, 4, 4, 33, 33, 32),
    (1, 2, 1, 5, 1, 256),    # kv_len = 1
]


@pytest.mark.parametrize("shape", SHAPES)
def test_sdpa_matches_bruteforce_c(shape):
    B, H_q, H_kv, q, kv, D = shape
    Q = _rand((B, H_q, q, D), 1)
    K = _rand((B, H_kv, kv, D), 2)
    V = _rand((B, H_kv, kv, D), 3)
    O, M, L = orc.sdpa(Q, K, V)
    Oc, Mc, Lc = c_oracle.cpu_attn(Q, K, V, dtype=np.float64)
    np.testing.assert_allclose(O, Oc, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(M, Mc, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(L, Lc, rtol=1e-12)
    O32, _, _ = orc.sdpa(Q.astype(np.float32), K.astype(np.float32), V.astype(np.float32),
                        acc=np.float32)
    Oc32, _, _ = c_oracle.cpu_attn(Q, K, V, dtype=np.float32)
    np.testing.assert_allclose(O32, Oc32, rtol=1e-4, atol=2e-6)


@pytest.mark.parametrize("shape", SHAPES)
def test_sdpa_matches_torch_cpu_sdpa(shape):
    torch = pytest.importorskip("torch")
    B, H_q, H_kv, q, kv, D = shape
    Q = _rand((B, H_q, q, D), 4)
    K = _rand((B, H_kv, kv, D), 5)
    V = _rand((B, H_kv, kv, D), 6)
    r = H_q // H_kv
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(Q), torch.from_numpy(K).repeat_interleave(r, dim=1),
        torch.from_numpy(V).repeat_interleave(r, dim=1)).numpy()
    O, _, _ = orc.sdpa(Q, K, V)
    np.testing.assert_allclose(O, ref, rtol=1e-11, atol=1e-12)


def test_sdpa_reference_style_fp32_matches_sdpa():
    Q, K, V = (x.astype(np.float32) for x in orc.normal_fp16_inputs(1, 8, 2, 64, 64, 128, 9))
    O = orc.sdpa_fp32_reference_style(Q, K, V)
    ref, _, _ = orc.sdpa(Q, K, V)
    np.testing.assert_allclose(O, ref, atol=5e-6)


# ---------------------------------------------------------------------------
# Closed forms and invariants
# ---------------------------------------------------------------------------
def test_closed_form_kv_len_one():
    Q, K, V = _rand((2, 4, 3, 64), 1), _rand((2, 2, 1, 64), 2), _rand((2, 2, 1, 64), 3)
    O, M, L = orc.sdpa(Q, K, V)
    np.testing.assert_array_equal(O, np.repeat(V, 2, axis=1).repeat(3, axis=2))
    np.testing.assert_array_equal(L, np.ones_like(L))
    np.testing.assert_allclose(M, np.einsum("bhqd,bhkd->bhq", Q, np.repeat(K, 2, axis=1)) / 8.0)


def test_closed_form_zero_query_gives_mean_of_v():
    Q = np.zeros((1, 2, 4, 32))
    K, V = _rand((1, 1, 10, 32), 1), _rand((1, 1, 10, 32), 2)
    O, M, L = orc.sdpa(Q, K, V)
    np.testing.assert_allclose(O, np.broadcast_to(V.mean(axis=2, keepdims=True), O.shape), atol=1e-15)
    np.testing.assert_array_equal(M, np.zeros_like(M))
    np.testing.assert_array_equal(L, np.full_like(L, 10.0))


def test_closed_form_identical_keys_give_mean_of_v():
    K = np.repeat(_rand((1, 1, 1, 16), 1), 12, axis=2)
    V = _rand((1, 1, 12, 16), 2)
    O, _, L = orc.sdpa(_rand((1, 1, 5, 16), 3), K, V)
    np.testing.assert_allclose(O, np.broadcast_to(V.mean(axis=2, keepdims=True), O.shape), atol=1e-14)
    np.testing.assert_allclose(L, 12.0)


def test_closed_form_dominant_score_selects_row():
    D = 64
    K = _rand((1, 1, 20, D), 1) * 0.01
    Q = np.zeros((1, 1, 1, D))
    Q[..., 0] = 1000.0
    K[0, 0, 13, 0] = 10.0   # score 10000/8 above the rest
    V = _rand((1, 1, 20, D), 2)
    O, _, _ = orc.sdpa(Q, K, V)
    np.testing.assert_allclose(O[0, 0, 0], V[0, 0, 13], atol=1e-12)


def test_invariant_gqa_equals_repeated_mha():
    Q, K, V = _rand((2, 8, 5, 32), 1), _rand((2, 2, 7, 32), 2), _rand((2, 2, 7, 32), 3)
    O, M, L = orc.sdpa(Q, K, V)
    O2, M2, L2 = orc.sdpa(Q, np.repeat(K, 4, axis=1), np.repeat(V, 4, axis=1))
    np.testing.assert_array_equal(O, O2)


def test_invariant_joint_kv_permutation():
    Q, K, V = _rand((1, 4, 6, 64), 1), _rand((1, 2, 50, 64), 2), _rand((1, 2, 50, 64), 3)
    perm = np.random.default_rng(0).permutation(50)
    O, M, L = orc.sdpa(Q, K, V)
    O2, M2, L2 = orc.sdpa(Q, K[:, :, perm], V[:, :, perm])
    np.testing.assert_allclose(O, O2, atol=1e-14)
    np.testing.assert_allclose(L, L2, rtol=1e-14)


def test_invariant_convex_combination_bounds():
    Q, K, V = _rand((1, 4, 30, 16), 1) * 3, _rand((1, 1, 40, 16), 2) * 3, _rand((1, 1, 40, 16), 3)
    O, _, L = orc.sdpa(Q, K, V)
    assert (O >= V.min(axis=2, keepdims=True) - 1e-12).all()
    assert (O <= V.max(axis=2, keepdims=True) + 1e-12).all()
    assert (L >= 1.0).all() and (L <= 40.0).all()


# ---------------------------------------------------------------------------
# Tiled model and split-KV merge
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("D", [16, 64, 128])
def test_tiled_model_reference_smoke_shapes(D):
    """kernel_models/flash_attn.py:269-281: seed 42, B=1, S=16, H_q=2,
    H_kv=1, max-abs < 1e-4 against SDPA."""
    rng = np.random.RandomState(42)
    Q = rng.randn(1, 2, 16, D).astype(np.float32)
    K = rng.randn(1, 1, 16, D).astype(np.float32)
    V = rng.randn(1, 1, 16, D).astype(np.float32)
    O, M, L = orc.tiled_online_softmax(Q, K, V, kv_block_rows=16)
    ref, Mr, Lr = orc.sdpa(Q, K, V)
    assert np.abs(O - ref).max() < 1e-4
    np.testing.assert_allclose(M, Mr, atol=1e-5)
    np.testing.assert_allclose(L, Lr, rtol=1e-5)


@pytest.mark.parametrize("S,blk", [(129, 128), (255, 128), (40, 16), (17, 8)])
def test_tiled_model_ragged_tiles(S, blk):
    Q, K, V = (x.astype(np.float32) for x in orc.normal_fp16_inputs(1, 4, 2, S, S, 64, S))
    O, _, _ = orc.tiled_online_softmax(Q, K, V, kv_block_rows=blk)
    ref, _, _ = orc.sdpa(Q, K, V)
    assert np.abs(O - ref).max() < 1e-5


@pytest.mark.parametrize("n_splits", [1, 2, 3, 7, 64])
def test_split_combine_equals_sdpa(n_splits):
    kv = 64
    Q, K, V = _rand((2, 4, 3, 32), 1), _rand((2, 2, kv, 32), 2), _rand((2, 2, kv, 32), 3)
    b = orc.split_bounds(kv, n_splits)
    assert b[0][0] == 0 and b[-1][1] == kv and all(x[1] == y[0] for x, y in zip(b, b[1:]))
    O, M, L = orc.split_kv_combine(*orc.split_kv_partials(Q, K, V, b))
    ref, Mr, Lr = orc.sdpa(Q, K, V)
    np.testing.assert_allclose(O, ref, atol=1e-13)
    np.testing.assert_allclose(M, Mr, atol=1e-14)
    np.testing.assert_allclose(L, Lr, rtol=1e-13)


def test_split_combine_with_empty_split():
    Q, K, V = _rand((1, 2, 2, 16), 1), _rand((1, 1, 10, 16), 2), _rand((1, 1, 10, 16), 3)
    bounds = [(0, 4), (4, 4), (4, 10)]
    O, _, _ = orc.split_kv_combine(*orc.split_kv_partials(Q, K, V, bounds))
    np.testing.assert_allclose(O, orc.sdpa(Q, K, V)[0], atol=1e-14)


# ---------------------------------------------------------------------------
# Planted mistakes: each plausible oracle bug must fail the independent checks.
# ---------------------------------------------------------------------------
def _sdpa_mutant(Q, K, V, kind):
    B, H_q, q_len, D = Q.shape
    H_kv = K.shape[1]
    ratio = H_q // H_kv
    O = np.empty_like(Q)
    for b in range(B):
        for h in range(H_q):
            hk = (h % H_kv) if kind == "gqa_modulo" else h // ratio
            s = Q[b, h] @ K[b, hk].T
            if kind != "no_scale":
                s = s / np.sqrt(D)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            if kind == "no_normalise":
                O[b, h] = p @ V[b, hk]
            elif kind == "v_transposed":
                O[b, h] = (p / p.sum(axis=1, keepdims=True)) @ V[b, hk][::-1]
            else:
                O[b, h] = (p / p.sum(axis=1, keepdims=True)) @ V[b, hk]
    return O


@pytest.mark.parametrize("kind", ["gqa_modulo", "no_scale", "no_normalise", "v_transposed"])
def test_planted_mistakes_are_caught(kind):
    Q, K, V = _rand((1, 8, 4, 32), 11), _rand((1, 2, 9, 32), 12), _rand((1, 2, 9, 32), 13)
    Oc, _, _ = c_oracle.cpu_attn(Q, K, V)
    bad = _sdpa_mutant(Q, K, V, kind)
    assert np.abs(bad - Oc).max() > 1e-3, f"mutant {kind} slipped through"
    good, _, _ = orc.sdpa(Q, K, V)
    assert np.abs(good - Oc).max() < 1e-12


def test_tolerance_metric():
    ref = np.ones((4, 4))
    ok, mx, rel = orc.within_tolerance(ref + 1e-3, ref)
    assert ok and abs(mx - 1e-3) < 1e-12
    ok, _, _ = orc.within_tolerance(ref + 3e-3, ref)
    assert not ok


def test_flops_and_bytes_formulas():
    # tests/bench_flash_attn.cu:125-131 at the headline configs.
    assert orc.attn_flops(1, 32, 4096, 4096, 128) == 274877906944
    assert orc.attn_bytes(1, 32, 8, 1, 4096, 128) == 16801792
    assert orc.attn_bytes(32, 32, 8, 1, 8192, 128) == 1074528256


# ---------------------------------------------------------------------------
# Key masking (causal, per-sequence key counts): the semantics of
# kf_attn_fwd_ex, pinned against the already-pinned unmasked sdpa on
# truncated inputs, torch's own causal attention, and closed forms.
# ---------------------------------------------------------------------------
def test_key_limits_closed_forms():
    np.testing.assert_array_equal(orc.key_limits(4, 4, causal=True)[0], [1, 2, 3, 4])
    np.testing.assert_array_equal(orc.key_limits(3, 5, causal=True)[0], [3, 4, 5])
    np.testing.assert_array_equal(orc.key_limits(5, 3, causal=True)[0], [0, 0, 1, 2, 3])
    np.testing.assert_array_equal(orc.key_limits(2, 9, kv_lens=[4, 0, 99], B=3),
                                  [[4, 4], [0, 0], [9, 9]])
    np.testing.assert_array_equal(orc.key_limits(3, 9, causal=True, kv_lens=[2, 9], B=2),
                                  [[0, 1, 2], [7, 8, 9]])
    np.testing.assert_array_equal(orc.key_limits(1, 7, causal=True)[0], [7])  # decode: no-op


@pytest.mark.parametrize("q_len,kv_len", [(6, 6), (4, 9), (7, 3)])
def test_causal_rows_equal_attention_over_their_prefix(q_len, kv_len):
    Q, K, V = _rand((1, 4, q_len, 16), 21), _rand((1, 2, kv_len, 16), 22), _rand((1, 2, kv_len, 16), 23)
    O, M, L = orc.sdpa(Q, K, V, causal=True)
    for i in range(q_len):
        n = i + kv_len - q_len + 1
        if n <= 0:
            assert (O[:, :, i] == 0).all() and np.isneginf(M[:, :, i]).all() and (L[:, :, i] == 0).all()
            continue
        Op, Mp, Lp = orc.sdpa(Q[:, :, i:i + 1], K[:, :, :n], V[:, :, :n])
        np.testing.assert_allclose(O[:, :, i:i + 1], Op, rtol=1e-13, atol=1e-15)
        np.testing.assert_allclose(M[:, :, i:i + 1], Mp, rtol=1e-13)
        np.testing.assert_allclose(L[:, :, i:i + 1], Lp, rtol=1e-13)


def test_causal_first_row_is_v0():
    Q, K, V = _rand((2, 4, 5, 32), 31), _rand((2, 4, 5, 32), 32), _rand((2, 4, 5, 32), 33)
    O, _, L = orc.sdpa(Q, K, V, causal=True)
    np.testing.assert_array_equal(O[:, :, 0], V[:, :, 0])
    np.testing.assert_array_equal(L[:, :, 0], 1.0)


@pytest.mark.parametrize("q_len,kv_len", [(8, 8), (5, 11)])
def test_causal_matches_torch(q_len, kv_len):
    torch = pytest.importorskip("torch")
    Q, K, V = _rand((2, 4, q_len, 16), 41), _rand((2, 2, kv_len, 16), 42), _rand((2, 2, kv_len, 16), 43)
    tq = torch.from_numpy(Q)
    tk = torch.from_numpy(K).repeat_interleave(2, dim=1)
    tv = torch.from_numpy(V).repeat_interleave(2, dim=1)
    if q_len == kv_len:
        ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    else:  # bottom-right alignment as a boolean tril mask
        mask = torch.ones(q_len, kv_len, dtype=torch.bool).tril(diagonal=kv_len - q_len)
        ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask)
    O, _, _ = orc.sdpa(Q, K, V, causal=True)
    np.testing.assert_allclose(O, ref.numpy(), rtol=1e-11, atol=1e-12)


def test_kv_lens_equal_truncated_sequences():
    Q, K, V = _rand((3, 4, 6, 16), 51), _rand((3, 2, 10, 16), 52), _rand((3, 2, 10, 16), 53)
    lens = [10, 1, 0]
    O, M, L = orc.sdpa(Q, K, V, kv_lens=lens)
    for b, n in enumerate(lens):
        if n == 0:
            assert (O[b] == 0).all() and np.isneginf(M[b]).all() and (L[b] == 0).all()
            continue
        Ob, Mb, Lb = orc.sdpa(Q[b:b + 1], K[b:b + 1, :, :n], V[b:b + 1, :, :n])
        np.testing.assert_allclose(O[b:b + 1], Ob, rtol=1e-13, atol=1e-15)
        np.testing.assert_allclose(M[b:b + 1], Mb, rtol=1e-13)
    # kv_len = 1 keeps the closed form O = V_0.
    O1, _, _ = orc.sdpa(Q, K, V, kv_lens=[1, 1, 1])
    np.testing.assert_array_equal(O1, np.repeat(V[:, :, :1], 2, axis=1).repeat(6, axis=2))


def test_planted_mask_off_by_one_is_caught(monkeypatch):
    real = orc.key_limits

    def shifted(*a, **kw):
        return np.maximum(real(*a, **kw) - 1, 0)

    monkeypatch.setattr(orc, "key_limits", shifted)
    Q, K, V = _rand((1, 2, 5, 16), 61), _rand((1, 2, 5, 16), 62), _rand((1, 2, 5, 16), 63)
    O, _, _ = orc.sdpa(Q, K, V, causal=True)
    assert not np.array_equal(O[:, :, 0], V[:, :, 0]), "off-by-one mask slipped through"


# ---------------------------------------------------------------------------
# Paged K/V cache: the gather restated two ways, and key validity.
# ---------------------------------------------------------------------------
def test_paged_gather_matches_reference_style_torch_gather():
    """bench_flash_attn2.py:190-196 gathers with K_pool[blk_ids].permute(1, 0,
    2, 3).reshape(H_kv, padded, D); per sequence that must equal the oracle."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    num_pages, H_kv, ps, D, B, max_pages = 12, 2, 16, 8, 2, 5
    pool = rng.standard_normal((num_pages, H_kv, ps, D))
    table = np.stack([rng.permutation(num_pages)[:max_pages] for _ in range(B)])
    K, valid = orc.paged_to_contiguous(pool, table, ps)
    assert valid.all()
    for b in range(B):
        ids = torch.from_numpy(table[b].astype(np.int64))
        g = torch.from_numpy(pool)[ids].permute(1, 0, 2, 3).reshape(H_kv, max_pages * ps, D)
        np.testing.assert_array_equal(K[b], g.numpy())


def test_paged_identity_table_is_contiguous_and_invalid_ids_drop_keys():
    rng = np.random.default_rng(6)
    B, H_kv, max_pages, ps, D = 2, 2, 3, 16, 8
    Kc = rng.standard_normal((B, H_kv, max_pages * ps, D))
    # Pool page b * max_pages + p holds rows [p*ps, (p+1)*ps) of sequence b.
    pool = Kc.reshape(B, H_kv, max_pages, ps, D).transpose(0, 2, 1, 3, 4).reshape(-1, H_kv, ps, D)
    table = np.arange(B * max_pages).reshape(B, max_pages)
    K, valid = orc.paged_to_contiguous(pool, table, ps)
    np.testing.assert_array_equal(K, Kc)
    table[1, 1] = -1
    table[0, 2] = B * max_pages
    _, valid = orc.paged_to_contiguous(pool, table, ps)
    assert not valid[1, ps:2 * ps].any() and not valid[0, 2 * ps:].any()
    assert valid.sum() == B * max_pages * ps - 2 * ps


def test_sdpa_key_valid_equals_dropping_the_keys():
    Q, K, V = _rand((2, 4, 3, 16), 71), _rand((2, 2, 20, 16), 72), _rand((2, 2, 20, 16), 73)
    valid = np.ones((2, 20), dtype=bool)
    valid[0, 5:9] = False
    valid[1, :] = False
    valid[1, 19] = True
    O, M, L = orc.sdpa(Q, K, V, key_valid=valid)
    keep = np.flatnonzero(valid[0])
    O0, M0, L0 = orc.sdpa(Q[:1], K[:1, :, keep], V[:1, :, keep])
    np.testing.assert_allclose(O[:1], O0, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(M[:1], M0, rtol=1e-13)
    # One valid key: O = that V row (closed form).
    np.testing.assert_array_equal(O[1], np.repeat(V[1, :, 19:20], 2, axis=0).repeat(3, axis=1))
    Oe, Me, Le = orc.sdpa(Q, K, V, key_valid=np.zeros((2, 20), dtype=bool))
    assert (Oe == 0).all() and np.isneginf(Me).all() and (Le == 0).all()
