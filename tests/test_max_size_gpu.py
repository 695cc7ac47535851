"""GPU check at the largest key count the ABI accepts (kv_len * D just under
2^31 elements per head: 4.3 GB each of K and V at D = 128), where element
offsets fill 31 bits and byte offsets reach 2^32.  Closed form, no oracle
run: every key is zero except the last one, whose score exceeds all others
by ~90 (e^-90 underflows the fp16 P to 0), so every output row must equal
the last V row exactly, while every other V row holds -1; Mi must be that
score and Li exactly 1.  A wrapped or truncated offset would read another
row and show up as -1 / a wrong Mi.  Run through the decode kernels, the
(65792 / 32896 query rows) the wide prefill kernel at D = 128 and 256, and
(64 rows) the split prefill, whose last KV partition holds the last key,
each unmasked and masked (key count = kv_len)."""
import math

import pytest
import torch

import kernelfoundry_amd as kf

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("q_len,H_q,D", [(1, 8, 128), (64, 1, 128), (1, 8, 256), (64, 1, 256),
                                         (2056, 32, 128), (1028, 32, 256)])
def test_last_key_at_the_offset_limit(q_len, H_q, D):
    kv = (2 ** 31 - 1) // D // 64 * 64 - 64
    names = kf.kernel_names(1, q_len, kv, H_q, 1, D)
    print("case", dict(q_len=q_len, H_q=H_q, D=D, kv=kv, path=kf.plan(1, q_len, kv, H_q, 1, D).path,
                       kernels=names), flush=True)
    # 65792 / 32896 rows: the wide prefill kernel; 64 rows: the split prefill
    wide = q_len > 1000
    split = q_len == 64
    masked = kf.kernel_names(1, q_len, kv, H_q, 1, D, masked=True)
    if wide:
        assert names == f"kf_attn_prefill_wide_kernel<{D}, false, 1, false>", names
        # ... and its masked instantiation, with the key count set to kv_len
        assert masked == f"kf_attn_prefill_wide_kernel<{D}, true, 1, false>", masked
    if split:
        assert kf.plan(1, q_len, kv, H_q, 1, D).path == "prefill_split"
        kern = "kf_attn_prefill_parts_kernel<256, " if D == 256 else f"kf_attn_prefill_kernel<{D}, "
        assert names.startswith(kern + "false") and "split_merge" in names
        assert masked.startswith(kern + "true") and "split_merge" in masked
    dev = torch.device("cuda")
    K = torch.zeros((1, 1, kv, D), dtype=torch.float16, device=dev)
    V = torch.full((1, 1, kv, D), -1.0, dtype=torch.float16, device=dev)
    K[0, 0, -1] = 16.0
    vlast = (torch.arange(D, device=dev, dtype=torch.float32) / D).half()
    V[0, 0, -1] = vlast
    Q = torch.full((1, H_q, q_len, D), 0.5, dtype=torch.float16, device=dev)
    try:
        runs = [None] + ([torch.tensor([kv], dtype=torch.int32, device=dev)] if wide or split else [])
        for lens in runs:
            O, Mi, Li = kf.attn_fwd(Q, K, V, return_stats=True, kv_lens=lens)
            torch.cuda.synchronize()
            want = vlast.float().expand(1, H_q, q_len, D)
            assert torch.equal(O, want), (lens is not None, (O - want).abs().max().item())
            score = 0.5 * 16.0 * D / math.sqrt(D)      # q.k / sqrt(D)
            assert torch.allclose(Mi, torch.full_like(Mi, score), rtol=1e-6, atol=1e-4)
            assert torch.equal(Li, torch.ones_like(Li))
            del O, Mi, Li
    finally:
        del K, V
        torch.cuda.empty_cache()


def test_last_row_at_the_offset_limit():
    """The same at the largest accepted query-row count (q_len * D just under
    2^31: 4.3 GB of Q, 8.6 GB of fp32 O): every row must equal the last V
    row, checked on the first, middle and last rows written."""
    D, kv = 128, 64
    q = (2 ** 31 - 1) // D // 256 * 256 - 256
    print("case", dict(q_len=q, D=D, kv=kv, path=kf.plan(1, q, kv, 1, 1, D).path), flush=True)
    dev = torch.device("cuda")
    K = torch.zeros((1, 1, kv, D), dtype=torch.float16, device=dev)
    V = torch.full((1, 1, kv, D), -1.0, dtype=torch.float16, device=dev)
    K[0, 0, -1] = 16.0
    vlast = (torch.arange(D, device=dev, dtype=torch.float32) / D).half()
    V[0, 0, -1] = vlast
    Q = torch.full((1, 1, q, D), 0.5, dtype=torch.float16, device=dev)
    try:
        O = kf.attn_fwd(Q, K, V)
        torch.cuda.synchronize()
        for rows in (slice(0, 1024), slice(q // 2, q // 2 + 1024), slice(q - 1024, q)):
            got = O[0, 0, rows]
            assert torch.equal(got, vlast.float().expand_as(got)), rows
        assert torch.equal(O[0, 0, :, 0], torch.zeros(q, device=dev))  # column 0 of vlast
    finally:
        del Q
        torch.cuda.empty_cache()


def test_paged_pool_with_the_largest_page_offsets():
    """Paged decode over a 4.3 GB page pool (2^20 pages of 16 rows, D = 128)
    with the block table in reverse page order: the dominant key sits on the
    highest page id, whose base offset is the largest, and must be the one
    that every output row equals."""
    D, ps = 128, 16
    pages = (2 ** 31 - 1) // D // ps - 8          # key capacity within 31 bits
    dev = torch.device("cuda")
    Kp = torch.zeros((pages, 1, ps, D), dtype=torch.float16, device=dev)
    Vp = torch.full((pages, 1, ps, D), -1.0, dtype=torch.float16, device=dev)
    top, row = pages - 1, 5                        # highest page id, a row inside it
    Kp[top, 0, row] = 16.0
    vhit = (torch.arange(D, device=dev, dtype=torch.float32) / D).half()
    Vp[top, 0, row] = vhit
    table = torch.arange(pages - 1, -1, -1, dtype=torch.int32, device=dev).reshape(1, pages)
    lens = torch.full((1,), pages * ps, dtype=torch.int32, device=dev)
    Q = torch.full((1, 8, 1, D), 0.5, dtype=torch.float16, device=dev)
    print("case", dict(pages=pages, keys=pages * ps), flush=True)
    try:
        O = kf.attn_decode_paged(Q, Kp, Vp, table, lens)
        torch.cuda.synchronize()
        assert torch.equal(O, vhit.float().expand_as(O)), (O - vhit.float()).abs().max().item()
    finally:
        del Kp, Vp
        torch.cuda.empty_cache()
