"""Seeded random-shape parity sweep of kf_attn_decode_paged on the GPU.

Each case draws the head dimension (16 / 64 / 128 / 256), the GQA ratio,
up to 32 query rows per KV head, the batch, the page size (16 .. 128), a
random placement of every sequence's pages in a larger pool, about 5 % of
block-table entries outside [0, num_pages) (negative, num_pages, far out of
range: those pages hold no keys), a key count per sequence from 0 to the
table's capacity, and causal masking in 30 % of the cases.  The result is
compared with the oracle's page gather (the layout of
reference_benchmarks/bench_flash_attn2.py:153-215) followed by its fp64
``sdpa`` on the same fp16 inputs, at the north-star bar (max |got - ref| <=
2e-3, ||got - ref|| / ||ref|| <= 1e-2; Mi to 1e-4, Li to 1e-3 relative;
rows without keys exactly O = 0, Mi = -inf, Li = 0).
"""
import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu


def _cases(n=40, seed=31337):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rng.choice([16, 64, 128, 256]))
        H_kv = int(rng.choice([1, 2, 4, 8]))
        ratio = int(rng.choice([1, 2, 4, 8]))
        q_len = int(rng.integers(1, 32 // ratio + 1))
        B = int(rng.integers(1, 9))
        ps = int(rng.choice([16, 32, 64, 128]))
        max_pages = int(rng.integers(1, max(2, 3000 // ps)))
        num_pages = int(B * max_pages * rng.uniform(1.0, 2.0)) + 1
        causal = bool(rng.random() < 0.3)
        out.append((B, H_kv * ratio, H_kv, q_len, D, ps, max_pages, num_pages, causal,
                    int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "B%d_Hq%d_Hkv%d_q%d_D%d_ps%d_mp%d_np%d_%s" % (
    *c[:8], "causal" if c[8] else "full"))
def test_paged_random(case):
    import torch

    import kernelfoundry_amd as kf

    B, H_q, H_kv, q_len, D, ps, max_pages, num_pages, causal, seed = case
    print("case", case, flush=True)
    g = np.random.default_rng(seed)
    table = g.permutation(num_pages)[:B * max_pages].reshape(B, max_pages).astype(np.int32)
    bad = g.random(table.shape) < 0.05
    table[bad] = g.choice([-1, num_pages, num_pages + 7, -(1 << 30)], size=int(bad.sum()))
    lens = g.integers(0, max_pages * ps + 1, size=B).astype(np.int32)
    q16 = g.standard_normal((B, H_q, q_len, D)).astype(np.float16)
    kp = g.standard_normal((num_pages, H_kv, ps, D)).astype(np.float16)
    vp = g.standard_normal((num_pages, H_kv, ps, D)).astype(np.float16)

    def dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).cuda()

    O, Mi, Li = kf.attn_decode_paged(dev(q16), dev(kp), dev(vp), dev(table), dev(lens),
                                     return_stats=True, causal=causal)
    torch.cuda.synchronize()
    O, Mi, Li = O.cpu().numpy(), Mi.cpu().numpy(), Li.cpu().numpy()

    K, valid = orc.paged_to_contiguous(kp, table, ps)
    V, _ = orc.paged_to_contiguous(vp, table, ps)
    Or, Mr, Lr = orc.sdpa(q16, K, V, causal=causal, kv_lens=[int(x) for x in lens],
                          key_valid=valid)
    assert np.isfinite(O).all(), "non-finite O"
    ok, max_abs, rel = orc.within_tolerance(O, Or)
    assert ok, f"max_abs={max_abs:.3g} rel={rel:.3g}"
    empty = np.isneginf(Mr)
    assert np.array_equal(np.isneginf(Mi), empty), "Mi = -inf on the wrong rows"
    assert (O[empty] == 0).all() and (Li[empty] == 0).all(), "empty rows not zero"
    full = ~empty
    if full.any():
        assert np.abs(Mi[full] - Mr[full]).max() <= 1e-4, "Mi"
        rel_l = np.abs(Li[full] - Lr[full]).max() / np.abs(Lr[full]).max()
        assert rel_l <= 1e-3, f"Li rel err {rel_l:.3g}"
