"""GPU checks of the output formats of kf_attn_fwd_ex / kf_attn_decode_paged:
fp16 and bf16 O, and the LSE row statistic.

The kernels compute O in fp32 and round only at the store, so an fp16 / bf16
O must equal the round-to-nearest-even of the fp32 O of the same call
configuration bit for bit (numpy's float16 cast and an explicit bf16 RNE on
the bits are the references).  LSE must equal Mi + ln(Li) of the fp32 call
(to the accuracy of the hardware log) and the fp64 oracle's
Mi + ln(Li) to 1e-3; rows without keys give LSE = -inf.

Every kernel path that writes O is covered: prefill (unmasked and masked, the
256-row and the wide kernel, masked by key counts and, at D = 256, causal;
the KV-group merges of both kernels; the split prefill, whose O the merge
kernel writes), decode without split (O written by the decode kernel), decode with split
(O written by the merge kernel), and paged decode.
"""
import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return torch


def _announce(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _bf16_rne(x32):
    u = np.ascontiguousarray(x32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


CASES = [
    # B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens       path
    (1, 8, 2, 300, 300, 128, False, None),                # prefill
    (32, 32, 8, 100, 77, 128, False, None),               # wide prefill (512-row workgroups)
    (2, 8, 2, 200, 260, 64, True, [260, 0]),              # prefill, masked, empty sequence
    (1, 4, 4, 64, 64, 256, False, None),                  # prefill D=256
    (4, 32, 8, 600, 777, 128, False, [777, 0, 31, 500]),  # wide prefill with key counts
    (4, 16, 4, 700, 500, 256, True, None),                # wide prefill D=256, causal, rows without keys
    (1, 16, 4, 300, 333, 256, False, None),               # wide prefill D=256, two KV groups (merge writes O)
    (1, 16, 4, 700, 500, 256, True, None),                # the same, causal, rows without keys
    (2, 16, 4, 300, 600, 256, False, [600, 31]),          # the same, key counts (one group without keys)
    (1, 8, 2, 128, 600, 128, False, None),                # prefill, four KV groups of 8 waves
    (2, 32, 8, 64, 3000, 128, True, [3000, 0]),           # split prefill (merge kernel writes O)
    (2, 32, 8, 40, 4096, 16, False, [4096, 100]),         # split prefill, one KV group per workgroup
    (2, 16, 4, 100, 3000, 256, True, None),               # split prefill at D=256 (4-wave kernel)
    (2, 8, 8, 1, 100, 16, False, None),                   # decode, one split
    (2, 32, 8, 1, 3000, 128, True, [3000, 7]),            # decode + merge kernel
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_q{}_kv{}_D{}".format(*c[:6]))
def test_output_formats_round_the_fp32_result(case):
    import kernelfoundry_amd as kf
    torch = _torch()
    B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens = case
    _announce(test="out_formats", B=B, H_q=H_q, H_kv=H_kv, q_len=q_len, kv_len=kv_len, D=D,
              causal=causal, kv_lens=kv_lens)
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, 555 + D)
    Q, K, V = (torch.from_numpy(x).cuda() for x in (q16, k16, v16))
    lens = None if kv_lens is None else torch.tensor(kv_lens, dtype=torch.int32, device="cuda")
    kw = dict(causal=causal, kv_lens=lens)
    O32, Mi, Li = kf.attn_fwd(Q, K, V, return_stats=True, **kw)
    O16 = kf.attn_fwd(Q, K, V, out_dtype=torch.float16, **kw)
    Obf, lse = kf.attn_fwd(Q, K, V, out_dtype=torch.bfloat16, return_lse=True, **kw)
    torch.cuda.synchronize()
    O32 = O32.cpu().numpy()
    assert O16.dtype == torch.float16 and Obf.dtype == torch.bfloat16
    np.testing.assert_array_equal(O16.cpu().numpy().view(np.uint16),
                                  O32.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(Obf.cpu().view(torch.int16).numpy().view(np.uint16),
                                  _bf16_rne(O32))
    Mi, Li, lse = Mi.cpu().numpy(), Li.cpu().numpy(), lse.cpu().numpy()
    empty = Li == 0
    assert np.isneginf(lse[empty]).all()
    full = ~empty
    np.testing.assert_allclose(lse[full], Mi[full] + np.log(Li[full]), rtol=0, atol=1e-5)
    _, Mr, Lr = orc.sdpa(q16, k16, v16, causal=causal, kv_lens=kv_lens)
    ref = Mr + np.log(np.where(Lr > 0, Lr, 1.0))
    assert np.abs(lse[full] - ref[full]).max() <= 1e-3


def test_paged_output_formats():
    import kernelfoundry_amd as kf
    torch = _torch()
    B, H_q, H_kv, D, ps, max_pages = 2, 32, 8, 128, 16, 40
    num_pages = B * max_pages
    _announce(test="paged_out_formats")
    rng = np.random.default_rng(77)
    f16 = lambda a: a.astype(np.float32).astype(np.float16)
    q16 = f16(rng.standard_normal((B, H_q, 1, D)))
    kp = f16(rng.standard_normal((num_pages, H_kv, ps, D)))
    vp = f16(rng.standard_normal((num_pages, H_kv, ps, D)))
    table = rng.permutation(num_pages).astype(np.int32).reshape(B, max_pages)
    lens = np.array([600, 17], dtype=np.int32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    args = (t(q16), t(kp), t(vp), t(table), t(lens))
    O32, Mi, Li = kf.attn_decode_paged(*args, return_stats=True)
    O16, lse = kf.attn_decode_paged(*args, out_dtype=torch.float16, return_lse=True)
    Obf = kf.attn_decode_paged(*args, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    O32 = O32.cpu().numpy()
    np.testing.assert_array_equal(O16.cpu().numpy().view(np.uint16),
                                  O32.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(Obf.cpu().view(torch.int16).numpy().view(np.uint16),
                                  _bf16_rne(O32))
    np.testing.assert_allclose(lse.cpu().numpy(), Mi.cpu().numpy() + np.log(Li.cpu().numpy()),
                               rtol=0, atol=1e-5)


def test_python_entries_reject_buffers_the_kernels_would_overrun():
    """A caller's O must match the shape and element size the kernels write
    (O defaults to fp32), a caller's workspace must be a device buffer and
    key counts must be contiguous: anything else raises before any launch."""
    import pytest
    import torch

    import kernelfoundry_amd as kf

    dev = torch.device("cuda")
    Q = torch.zeros((1, 4, 8, 64), dtype=torch.float16, device=dev)
    K = torch.zeros((1, 2, 16, 64), dtype=torch.float16, device=dev)
    V = torch.zeros_like(K)
    for bad in (torch.empty((1, 4, 8, 64), dtype=torch.float16, device=dev),   # fp16, fp32 written
                torch.empty((1, 4, 8, 32), dtype=torch.float32, device=dev),   # too few columns
                torch.empty((1, 8, 4, 64), dtype=torch.float32, device=dev).transpose(1, 2)):
        with pytest.raises(ValueError):
            kf.attn_fwd(Q, K, V, out=bad)
    with pytest.raises(ValueError):
        kf.attn_fwd(Q, K, V, out=torch.empty((1, 4, 8, 64), dtype=torch.float32, device=dev),
                    out_dtype=torch.bfloat16)
    Q1 = torch.zeros((1, 4, 1, 64), dtype=torch.float16, device=dev)
    K1 = torch.zeros((1, 2, 4096, 64), dtype=torch.float16, device=dev)
    assert kf.plan(1, 1, 4096, 4, 2, 64).workspace_bytes > 0
    with pytest.raises(ValueError):
        kf.attn_fwd(Q1, K1, K1, workspace=torch.empty(1 << 24, dtype=torch.uint8))
    # Key counts are read in the caller's layout: a strided view is rejected
    # (a copy made on another stream would be unordered with the launch).
    Q2 = torch.zeros((2, 4, 8, 64), dtype=torch.float16, device=dev)
    K2 = torch.zeros((2, 2, 16, 64), dtype=torch.float16, device=dev)
    strided = torch.full((4,), 8, dtype=torch.int32, device=dev)[::2]
    assert not strided.is_contiguous()
    with pytest.raises(ValueError):
        kf.attn_fwd(Q2, K2, K2, kv_lens=strided)
    # Paged decode: same rule for O.
    Kp = torch.zeros((8, 2, 16, 64), dtype=torch.float16, device=dev)
    table = torch.arange(8, dtype=torch.int32, device=dev).reshape(1, 8)
    lens = torch.full((1,), 100, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        kf.attn_decode_paged(Q1, Kp, Kp, table, lens,
                             out=torch.empty((1, 4, 1, 64), dtype=torch.float16, device=dev))
    # The well-formed calls still run.
    O = kf.attn_fwd(Q, K, V, out=torch.empty((1, 4, 8, 64), dtype=torch.float32, device=dev))
    O16 = kf.attn_decode_paged(Q1, Kp, Kp, table, lens, out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert torch.isfinite(O).all() and O16.dtype == torch.float16


def test_python_entries_on_a_side_stream():
    """attn_fwd / attn_decode_paged launched on a stream other than torch's
    current one (new O, Mi, Li and workspace allocated by the call) give the
    same bits as on the current stream."""
    import torch

    import kernelfoundry_amd as kf

    _announce(test="side_stream")
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    Q = torch.randn((2, 32, 1, 128), generator=g, device=dev).half()
    K = torch.randn((2, 8, 3000, 128), generator=g, device=dev).half()
    V = torch.randn((2, 8, 3000, 128), generator=g, device=dev).half()
    assert kf.plan(2, 1, 3000, 32, 8, 128).workspace_bytes > 0
    Kp = K[0].reshape(8, 3000 // 24, 24, 128)[:, :120, :16].permute(1, 0, 2, 3).contiguous()
    Vp = V[0].reshape(8, 3000 // 24, 24, 128)[:, :120, :16].permute(1, 0, 2, 3).contiguous()
    table = torch.arange(120, dtype=torch.int32, device=dev).flip(0).reshape(2, 60).contiguous()
    lens = torch.tensor([960, 513], dtype=torch.int32, device=dev)
    ref = kf.attn_fwd(Q, K, V, return_stats=True)
    ref_p = kf.attn_decode_paged(Q, Kp, Vp, table, lens, return_stats=True)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    got = kf.attn_fwd(Q, K, V, return_stats=True, stream=side)
    got_p = kf.attn_decode_paged(Q, Kp, Vp, table, lens, return_stats=True, stream=side)
    side.synchronize()
    for a, b in zip(ref + ref_p, got + got_p):
        assert torch.equal(a, b)


def test_side_stream_outputs_do_not_reuse_memory_busy_on_the_current_stream():
    """A tensor freed while a kernel queued on torch's current stream still
    writes it must not become the O of a launch on another stream: the call
    allocates O, Mi, Li and the workspace from the launch stream's pool.
    The current stream is held busy (a spin kernel) in front of a fill of a
    freed tensor of O's size; the side-stream result must equal the
    current-stream result bit for bit."""
    import torch

    import kernelfoundry_amd as kf

    _announce(test="side_stream_alloc")
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(9)
    Q = torch.randn((1, 32, 1, 128), generator=g, device=dev).half()
    K = torch.randn((1, 8, 4096, 128), generator=g, device=dev).half()
    V = torch.randn((1, 8, 4096, 128), generator=g, device=dev).half()
    assert kf.plan(1, 1, 4096, 32, 8, 128).workspace_bytes > 0
    ref, ref_m, ref_l = kf.attn_fwd(Q, K, V, return_stats=True)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=dev)
    cur = torch.cuda.current_stream(dev)
    for _ in range(3):
        X = torch.empty_like(ref)
        Xm = torch.empty_like(ref_m)
        Xw = torch.empty(kf.workspace_bytes(1, 1, 4096, 32, 8, 128), dtype=torch.uint8, device=dev)
        torch.cuda._sleep(20_000_000)       # keeps the current stream busy for ~10 ms
        X.fill_(7.0)
        Xm.fill_(7.0)
        Xw.fill_(7)
        del X, Xm, Xw                        # freed to the current stream's pool, still pending
        got, got_m, got_l = kf.attn_fwd(Q, K, V, return_stats=True, stream=side)
        side.synchronize()
        cur.synchronize()
        assert torch.equal(got, ref) and torch.equal(got_m, ref_m) and torch.equal(got_l, ref_l)
