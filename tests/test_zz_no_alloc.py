"""GPU checks of kf_attn_fwd_noalloc, the entry point that allocates nothing
(its split-KV partials live in the library's static per-device scratch).

Through the C ABI (ctypes), each case runs kf_attn_fwd_ex with a caller
workspace and kf_attn_fwd_noalloc on the same inputs and compares O, Mi and
Li bit for bit: both launch the same kernels, so the static scratch must
change nothing.  Two calls in a row, the second on a smaller input, check
that the second call is not disturbed by what the first left in the
scratch.  A shape needing more than the static maximum is refused with
KF_ERR_SCRATCH and launches nothing.
"""
import ctypes

import pytest

pytestmark = pytest.mark.gpu


def _announce(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return torch


def _inputs(torch, B, H_q, H_kv, q, kv, D, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q = torch.randn((B, H_q, q, D), generator=g, device="cuda").half()
    K = torch.randn((B, H_kv, kv, D), generator=g, device="cuda").half()
    V = torch.randn((B, H_kv, kv, D), generator=g, device="cuda").half()
    return Q, K, V


def _both(torch, kf, B, H_q, H_kv, q, kv, D, seed, flags=0, lens=None):
    lib = kf.load_library()
    Q, K, V = _inputs(torch, B, H_q, H_kv, q, kv, D, seed)
    kvl = None if lens is None else torch.tensor(lens, dtype=torch.int32, device="cuda")
    kvp = kvl.data_ptr() if kvl is not None else None
    need = kf.workspace_bytes(B, q, kv, H_q, H_kv, D)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
    outs = []
    for noalloc in (False, True):
        O = torch.full((B, H_q, q, D), float("nan"), device="cuda")
        Mi = torch.full((B, H_q, q), float("nan"), device="cuda")
        Li = torch.full((B, H_q, q), float("nan"), device="cuda")
        s = torch.cuda.current_stream().cuda_stream
        if noalloc:
            st = lib.kf_attn_fwd_noalloc(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(),
                                         Mi.data_ptr(), Li.data_ptr(), B, q, kv, H_q, H_kv, D,
                                         kvp, flags, s)
        else:
            st = lib.kf_attn_fwd_ex(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(),
                                    Mi.data_ptr(), Li.data_ptr(), B, q, kv, H_q, H_kv, D, kvp,
                                    flags, ws.data_ptr(), need, s)
        assert st == kf.KF_OK, kf.status_string(st)
        outs.append((O, Mi, Li))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    return need


@pytest.mark.parametrize("first,second", [
    # B, H_q, H_kv, q_len, kv_len, D, flags, kv_lens
    ((1, 32, 8, 1, 4096, 128, 0, None), (1, 32, 8, 1, 1000, 128, 0, None)),
    ((1, 32, 8, 4, 8192, 128, 1, [8000]), (2, 32, 8, 1, 3000, 128, 1, [3000, 77])),
    ((1, 32, 1, 1, 2048, 64, 0, None), (1, 16, 1, 1, 700, 64, 0, None)),
    ((1, 32, 8, 64, 4096, 128, 0, None), (1, 32, 8, 16, 2048, 128, 1, [1500])),
], ids=["c2_then_smaller", "causal_lens_then_smaller", "mqa_then_smaller",
        "split_prefill_then_smaller"])
def test_noalloc_equals_workspace_entry_on_two_calls(first, second):
    import kernelfoundry_amd as kf
    torch = _torch()
    lib = kf.load_library()
    scratch = lib.kf_attn_noalloc_scratch_bytes()
    assert scratch == 16 << 20
    sizes = []
    for i, (B, H_q, H_kv, q, kv, D, flags, lens) in enumerate((first, second)):
        _announce(test="noalloc", call=i, B=B, H_q=H_q, H_kv=H_kv, q=q, kv=kv, D=D, flags=flags,
                  kv_lens=lens)
        sizes.append(_both(torch, kf, B, H_q, H_kv, q, kv, D, 100 + i, flags, lens))
    assert 0 < sizes[1] < sizes[0] <= scratch


def test_noalloc_without_scratch_and_after_other_calls():
    """A prefill (no split-KV scratch) and then a split decode again: the
    entry point serves both, and the decode result still matches."""
    import kernelfoundry_amd as kf
    torch = _torch()
    _announce(test="noalloc_prefill")
    assert _both(torch, kf, 1, 8, 2, 300, 300, 128, 7) == 0
    _announce(test="noalloc_decode_again")
    assert _both(torch, kf, 1, 32, 8, 1, 4096, 128, 8) > 0


def test_noalloc_refuses_a_shape_beyond_its_scratch():
    import kernelfoundry_amd as kf
    torch = _torch()
    lib = kf.load_library()
    B, H_q, H_kv, q, kv, D = 1, 256, 8, 1, 8192, 128
    assert kf.workspace_bytes(B, q, kv, H_q, H_kv, D) > lib.kf_attn_noalloc_scratch_bytes()
    _announce(test="noalloc_oversize")
    Q, K, V = _inputs(torch, B, H_q, H_kv, q, kv, D, 3)
    O = torch.full((B, H_q, q, D), 5.0, device="cuda")
    st = lib.kf_attn_fwd_noalloc(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), None,
                                 None, B, q, kv, H_q, H_kv, D, None, 0,
                                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st == kf.KF_ERR_SCRATCH
    assert bool((O == 5.0).all())


def test_noalloc_split_prefill_takes_the_partitions_its_scratch_holds():
    """A split prefill whose full plan needs more partials than the static
    scratch is planned with fewer KV partitions instead of being refused:
    the call succeeds, allocates nothing, and agrees with the fp64 oracle
    to the north-star bar on sampled heads and with kf_attn_fwd_ex (whose
    plan has more partitions, so P is rounded to fp16 against other row
    maxima) to 2e-4."""
    import kernelfoundry_amd as kf
    torch = _torch()
    lib = kf.load_library()
    B, H_q, H_kv, q, kv, D = 1, 32, 8, 64, 4096, 256
    assert kf.plan(B, q, kv, H_q, H_kv, D).path == "prefill_split"
    assert kf.workspace_bytes(B, q, kv, H_q, H_kv, D) > lib.kf_attn_noalloc_scratch_bytes()
    _announce(test="noalloc_split_prefill_capped", B=B, q=q, kv=kv, D=D)
    Q, K, V = _inputs(torch, B, H_q, H_kv, q, kv, D, 11)
    ref = kf.attn_fwd(Q, K, V)
    O = torch.full((B, H_q, q, D), float("nan"), device="cuda")
    st = lib.kf_attn_fwd_noalloc(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), None,
                                 None, B, q, kv, H_q, H_kv, D, None, 0,
                                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st == kf.KF_OK, kf.status_string(st)
    assert torch.isfinite(O).all()
    assert (O - ref).abs().max().item() <= 2e-4
    from oracle import attn_oracle as orc
    q16, k16, v16 = (t.cpu().numpy() for t in (Q, K, V))
    On = O.cpu().numpy()
    for h in (0, 31):
        want, _, _ = orc.sdpa(q16[:, h:h + 1], k16[:, h // 4:h // 4 + 1], v16[:, h // 4:h // 4 + 1])
        ok, max_abs, rel = orc.within_tolerance(On[:, h:h + 1], want)
        assert ok, (h, max_abs, rel)


def _noalloc(lib, torch, Q, K, V, O, Mi, Li, flags=0):
    B, H_q, q, D = Q.shape
    H_kv, kv = K.shape[1], K.shape[2]
    return lib.kf_attn_fwd_noalloc(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(),
                                   Mi.data_ptr(), Li.data_ptr(), B, q, kv, H_q, H_kv, D, None,
                                   flags, torch.cuda.current_stream().cuda_stream)


# B, H_q, H_kv, q_len, kv_len, D: the configs[1] split decode and a split
# prefill, both of which put their partials in the static scratch.
_SCRATCH_SHAPES = ((1, 32, 8, 1, 4096, 128), (1, 32, 8, 64, 4096, 128))


def test_noalloc_allocates_no_device_memory():
    """Repeated calls leave torch's allocator and the device's free memory
    (hipMemGetInfo) exactly where they were, after one warm call per shape
    (which may load the library's code object)."""
    import kernelfoundry_amd as kf
    torch = _torch()
    lib = kf.load_library()
    bufs = []
    for i, (B, H_q, H_kv, q, kv, D) in enumerate(_SCRATCH_SHAPES):
        assert kf.workspace_bytes(B, q, kv, H_q, H_kv, D) > 0
        Q, K, V = _inputs(torch, B, H_q, H_kv, q, kv, D, 40 + i)
        O = torch.empty((B, H_q, q, D), device="cuda")
        Mi = torch.empty((B, H_q, q), device="cuda")
        Li = torch.empty((B, H_q, q), device="cuda")
        bufs.append((Q, K, V, O, Mi, Li))
        _announce(test="noalloc_warm", B=B, q=q, kv=kv, D=D)
        assert _noalloc(lib, torch, Q, K, V, O, Mi, Li) == kf.KF_OK
    torch.cuda.synchronize()
    alloc0 = torch.cuda.memory_allocated()
    free0, _ = torch.cuda.mem_get_info()
    _announce(test="noalloc_repeat")
    for _ in range(20):
        for b in bufs:
            assert _noalloc(lib, torch, *b) == kf.KF_OK
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == alloc0
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)


def test_noalloc_captured_in_a_graph_replays_the_eager_result():
    """kf_attn_fwd_noalloc captured into a HIP graph (torch.cuda.CUDAGraph on
    a side stream, after a warm eager call) replays bit for bit what the
    eager call computed, on every replay, with eager work and
    synchronisations between the replays."""
    import kernelfoundry_amd as kf
    torch = _torch()
    lib = kf.load_library()
    cases = []
    for i, (B, H_q, H_kv, q, kv, D) in enumerate(_SCRATCH_SHAPES):
        Q, K, V = _inputs(torch, B, H_q, H_kv, q, kv, D, 60 + i)
        outs = tuple(torch.empty(s, device="cuda") for s in ((B, H_q, q, D), (B, H_q, q), (B, H_q, q)))
        _announce(test="noalloc_graph_eager", B=B, q=q, kv=kv, D=D)
        assert _noalloc(lib, torch, Q, K, V, *outs) == kf.KF_OK
        torch.cuda.synchronize()
        cases.append(((Q, K, V), outs, tuple(t.clone() for t in outs)))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    _announce(test="noalloc_graph_capture")
    with torch.cuda.graph(g, stream=side):
        for qkv, outs, _ in cases:
            assert _noalloc(lib, torch, *qkv, *outs) == kf.KF_OK
    torch.cuda.synchronize()
    for rep in range(3):
        for _, outs, _ in cases:
            for t in outs:
                t.fill_(float("nan"))
        torch.cuda.synchronize()
        _announce(test="noalloc_graph_replay", replay=rep)
        g.replay()
        torch.cuda.synchronize()
        for _, outs, eager in cases:
            for a, b in zip(outs, eager):
                assert torch.equal(a, b), f"replay {rep} differs from the eager call"
    del g


_FIRST_CALL_IN_CAPTURE = r"""
import sys
sys.path.insert(0, {repo!r})
import torch
import kernelfoundry_amd as kf
lib = kf.load_library()
B, H_q, H_kv, q, kv, D = 1, 32, 8, 1, 4096, 128
g = torch.Generator(device="cuda").manual_seed(5)
Q = torch.randn((B, H_q, q, D), generator=g, device="cuda").half()
K = torch.randn((B, H_kv, kv, D), generator=g, device="cuda").half()
V = torch.randn((B, H_kv, kv, D), generator=g, device="cuda").half()
O = torch.empty((B, H_q, q, D), device="cuda")
torch.cuda.synchronize()
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
print("capture: first kf_attn_fwd_noalloc call of the process", flush=True)
with torch.cuda.graph(graph, stream=side):
    st = lib.kf_attn_fwd_noalloc(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), None,
                                 None, B, q, kv, H_q, H_kv, D, None, 0,
                                 torch.cuda.current_stream().cuda_stream)
assert st == kf.KF_OK, kf.status_string(st)
torch.cuda.synchronize()
need = kf.workspace_bytes(B, q, kv, H_q, H_kv, D)
ws = torch.empty(need, dtype=torch.uint8, device="cuda")
ref = torch.empty_like(O)
st = lib.kf_attn_fwd_ex(Q.data_ptr(), K.data_ptr(), V.data_ptr(), ref.data_ptr(), None, None,
                        B, q, kv, H_q, H_kv, D, None, 0, ws.data_ptr(), need,
                        torch.cuda.current_stream().cuda_stream)
assert st == kf.KF_OK
for rep in range(2):
    O.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(O, ref), rep
print("first-call-in-capture OK", flush=True)
"""


def test_noalloc_first_call_of_the_process_inside_a_capture():
    """In a fresh process whose first kf_attn_fwd_noalloc call (and so the
    resolution of the static scratch's address) happens inside a graph
    capture, the capture succeeds and its replays equal kf_attn_fwd_ex."""
    import os
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    _announce(test="noalloc_first_call_in_capture", process="child")
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE.format(repo=repo)],
                         capture_output=True, text=True, timeout=150)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0
    assert "first-call-in-capture OK" in res.stdout
