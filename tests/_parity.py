"""Shared GPU parity check of kf_attn_fwd_ex against the fp64 oracle (test
infrastructure): max |got - ref| <= 2e-3 and ||got - ref|| / ||ref|| <= 1e-2,
Mi to 1e-4, Li to 1e-3 relative, rows without keys exactly O = 0,
Mi = -inf, Li = 0."""
import numpy as np

from oracle import attn_oracle as orc


def run_and_check(B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, seed):
    import torch

    import kernelfoundry_amd as kf

    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    pl = kf.plan(B, q_len, kv_len, H_q, H_kv, D)
    print("case", (B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, seed), pl.path,
          pl.block_threads, pl.grid_blocks, pl.num_splits, flush=True)
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, seed)
    Q, K, V = (torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (q16, k16, v16))
    lens = None if kv_lens is None else torch.tensor(kv_lens, dtype=torch.int32, device="cuda")
    O, Mi, Li = kf.attn_fwd(Q, K, V, return_stats=True, causal=causal, kv_lens=lens)
    torch.cuda.synchronize()
    O, Mi, Li = O.cpu().numpy(), Mi.cpu().numpy(), Li.cpu().numpy()
    Or, Mr, Lr = orc.sdpa(q16, k16, v16, causal=causal, kv_lens=kv_lens)
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
