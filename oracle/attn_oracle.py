"""CPU oracle for the flash-attention forward.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``kernelfoundry_amd``,
``include/``) may import, link or call this module.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use it, and
only as the checker (or as the timed CPU baseline), never as the thing
measured on the GPU.

It restates, from the mathematics, the algorithm of the reference
(sviraaj/kernelfoundry) for the attention forward:

  * ``sdpa``            -- exact scaled-dot-product attention with GQA grouping,
                           in fp64 or fp32.  Semantics of
                           kernel_models/flash_attn.py:250-265 (``reference_attn``)
                           and tests/test_flash_attn.cu:119-169 (``cpu_attn``),
                           generalised to q_len != kv_len.  Also returns the row
                           statistics the reference kernel writes:
                           Mi = max_j s_ij and Li = sum_j exp(s_ij - Mi) over
                           scaled scores s = q.k / sqrt(D)
                           (kernels/flash_attn.cu:559-579).
  * ``tiled_online_softmax`` -- the tiled online-softmax model with the reference's
                           geometry (Br=16 query rows, Bc_col=8 key columns,
                           kv_block_rows=128; kernel_models/flash_attn.py:33-37,
                           87-246), vectorised over the 16 rows of a query tile.
                           Prefill only (q_len == kv_len), as in the reference.
  * ``split_kv_partials`` / ``split_kv_combine`` -- the flash-decoding identity
                           m = max_k m_k, l = sum_k l_k e^(m_k-m),
                           O = sum_k O_k l_k e^(m_k-m) / l.  The reference has no
                           split-KV path; this is the published flash-decoding
                           merge rule, used to check the GPU split-KV kernels.
  * input generators    -- ``normal_fp16_inputs`` (N(0,1) -> fp16 RNE, seeds s,
                           s+1, s+2 as tests/test_flash_attn.cu:238-240) and
                           ``mt19937_uniform_f32`` (bit-exact restatement of
                           tests/test_utils.h:27-31: std::mt19937 +
                           std::uniform_real_distribution<float> as implemented
                           by libstdc++'s generate_canonical).

Pinning (how each function is checked against something it does not restate;
the tests live in tests/test_oracle.py):
  * sdpa            -- brute-force C triple loop (oracle/cpu_attn.c, a
                       restatement of tests/test_flash_attn.cu:119-169),
                       torch's CPU scaled_dot_product_attention in fp64 (a
                       library routine), closed forms (KV_len=1 -> O=V_0;
                       Q=0 -> column means of V; one dominant score -> that V
                       row), invariants (GQA == MHA with repeat_interleave'd
                       K/V; joint permutation of K/V rows; convex-combination
                       bounds).  The reference ships no fixture files; its
                       one known-answer test (kernel_models/flash_attn.py:
                       269-281) is reproduced for tiled_online_softmax below.
  * tiled_online_softmax -- equals sdpa on the reference's own smoke shapes
                       (kernel_models/flash_attn.py:269-281: B=1, S=16, H_q=2,
                       H_kv=1, D in {16,64,128}, max-abs < 1e-4) and on ragged
                       multi-tile shapes.
  * split_kv_combine -- equals sdpa for every split count, including splits
                       of length 1 and uneven splits.
  * mt19937_uniform_f32 -- compared bit-for-bit with libstdc++'s
                       std::mt19937/std::uniform_real_distribution<float>
                       compiled from a tiny g++ program at test time.
"""
from __future__ import annotations

import math

import numpy as np

LOG2E = 1.4426950408889634


# ---------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------

def fp16_round(x: np.ndarray) -> np.ndarray:
    """Round to IEEE binary16 with round-to-nearest-even.

    Same conversion as ``__float2half`` in tests/test_flash_attn.cu:173-178.
    """
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, seed):
    """Q/K/V drawn i.i.d. N(0,1) and rounded to fp16.

    Seeds follow the reference test convention (tests/test_flash_attn.cu:238-240):
    Q from ``seed``, K from ``seed+1``, V from ``seed+2``.  Layout [B, H, S, D].
    """
    q = np.random.default_rng(seed).standard_normal((B, H_q, q_len, D), dtype=np.float32)
    k = np.random.default_rng(seed + 1).standard_normal((B, H_kv, kv_len, D), dtype=np.float32)
    v = np.random.default_rng(seed + 2).standard_normal((B, H_kv, kv_len, D), dtype=np.float32)
    return fp16_round(q), fp16_round(k), fp16_round(v)


def mt19937_uniform_f32(n: int, lo: float, hi: float, seed: int) -> np.ndarray:
    """Bit-exact ``fill_random_f32`` (tests/test_utils.h:27-31).

    std::mt19937(seed) is Matsumoto & Nishimura's MT19937 seeded with
    init_genrand, which is also what numpy's legacy RandomState(int) uses, so
    the raw 32-bit stream is read from there.  libstdc++'s
    uniform_real_distribution<float> draws one 32-bit word per value
    (generate_canonical<float, 24> needs ceil(24/32) = 1 word), computes
    u = float(word) / 2^32 in float, clamps u >= 1 to nextafter(1, 0), and
    returns u * (hi - lo) + lo evaluated in float.
    """
    rs = np.random.RandomState(seed & 0xFFFFFFFF)
    # The bit generator's raw 32-bit outputs, one word per value.
    raw = rs._bit_generator.random_raw(n).astype(np.uint64) & 0xFFFFFFFF
    u = raw.astype(np.float32) / np.float32(4294967296.0)
    u = np.where(u >= np.float32(1.0), np.nextafter(np.float32(1.0), np.float32(0.0)), u)
    u = u.astype(np.float32)
    span = np.float32(np.float32(hi) - np.float32(lo))
    return (u * span + np.float32(lo)).astype(np.float32)


def reference_case_inputs(B, S, H_q, H_kv, D, seed):
    """Inputs of one ``run_case`` of tests/test_flash_attn.cu:228-251.

    Returns the unrounded fp32 tensors (what ``cpu_attn`` sees, :245) and their
    fp16 roundings (what the GPU sees, :248-251).  Layout [B, H, S, D].
    """
    q = mt19937_uniform_f32(B * H_q * S * D, -1.0, 1.0, seed).reshape(B, H_q, S, D)
    k = mt19937_uniform_f32(B * H_kv * S * D, -1.0, 1.0, seed + 1).reshape(B, H_kv, S, D)
    v = mt19937_uniform_f32(B * H_kv * S * D, -1.0, 1.0, seed + 2).reshape(B, H_kv, S, D)
    return (q, k, v), (fp16_round(q), fp16_round(k), fp16_round(v))


# The 18 cases of tests/test_flash_attn.cu:295-318: (B, S, H_q, H_kv, D, seed).
REFERENCE_CASES = (
    (1, 16, 1, 1, 16, 100),
    (1, 16, 1, 1, 64, 101),
    (1, 64, 1, 1, 128, 102),
    (1, 17, 1, 1, 128, 103),
    (1, 129, 1, 1, 128, 202),
    (1, 255, 1, 1, 128, 203),
    (1, 256, 1, 1, 64, 200),
    (1, 256, 1, 1, 128, 201),
    (1, 64, 4, 2, 64, 300),
    (1, 64, 8, 2, 64, 301),
    (1, 64, 32, 8, 128, 302),
    (1, 64, 40, 8, 128, 303),
    (1, 64, 8, 1, 128, 304),
    (1, 16, 1, 1, 256, 305),
    (2, 64, 4, 4, 64, 400),
    (2, 128, 4, 2, 128, 401),
    (3, 33, 4, 4, 128, 402),
    (2, 129, 32, 8, 128, 403),
)
REFERENCE_TOL = 5e-2  # tests/test_flash_attn.cu:22 (against unrounded fp32 inputs)


# ---------------------------------------------------------------------------
# Exact attention
# ---------------------------------------------------------------------------

def _check_shapes(Q, K, V):
    B, H_q, q_len, D = Q.shape
    Bk, H_kv, kv_len, Dk = K.shape
    if K.shape != V.shape or Bk != B or Dk != D:
        raise ValueError(f"shape mismatch Q{Q.shape} K{K.shape} V{V.shape}")
    if H_q % H_kv != 0:
        raise ValueError("H_q must be a multiple of H_kv")
    return B, H_q, H_kv, q_len, kv_len, D


def key_limits(q_len, kv_len, causal=False, kv_lens=None, B=1):
    """Visible keys per (batch, query index): an int array [B, q_len].

    Sequence b uses its first kv_b = clip(kv_lens[b], 0, kv_len) keys (all
    kv_len when kv_lens is None); with ``causal`` query i sees keys
    j <= i + kv_b - q_len (bottom-right aligned), i.e. the first
    clip(i + kv_b - q_len + 1, 0, kv_b).  The semantics of kf_attn_fwd_ex;
    the reference has no masking (kernels/flash_attn.cu:384-585).
    """
    if kv_lens is None:
        kvb = np.full(B, kv_len, dtype=np.int64)
    else:
        kvb = np.clip(np.asarray(kv_lens, dtype=np.int64).reshape(B), 0, kv_len)
    lim = np.repeat(kvb[:, None], q_len, axis=1)
    if causal:
        i = np.arange(q_len, dtype=np.int64)[None, :]
        lim = np.clip(i + kvb[:, None] - q_len + 1, 0, kvb[:, None])
    return lim


def paged_to_contiguous(K_pages, block_table, page_size):
    """Gather a paged cache into per-sequence rows.

    K_pages [num_pages, H_kv, page_size, D], block_table int [B, max_pages]
    -> (K [B, H_kv, max_pages * page_size, D], key_valid bool [B, cap]):
    key j of sequence b is row j % page_size of page block_table[b, j //
    page_size] (the layout of reference_benchmarks/bench_flash_attn2.py:
    153-215); keys on a page id outside [0, num_pages) are invalid (zeros).
    """
    num_pages, H_kv, ps, D = K_pages.shape
    assert ps == page_size
    table = np.asarray(block_table)
    B, max_pages = table.shape
    cap = max_pages * page_size
    K = np.zeros((B, H_kv, cap, D), dtype=K_pages.dtype)
    valid = np.zeros((B, cap), dtype=bool)
    for b in range(B):
        for pg in range(max_pages):
            pid = int(table[b, pg])
            if 0 <= pid < num_pages:
                K[b, :, pg * page_size:(pg + 1) * page_size] = K_pages[pid]
                valid[b, pg * page_size:(pg + 1) * page_size] = True
    return K, valid


def sdpa(Q, K, V, acc=np.float64, causal=False, kv_lens=None, key_valid=None):
    """Exact attention with GQA grouping; returns (O, Mi, Li).

    h_kv = h_q // (H_q // H_kv) (kernels/flash_attn.cu:406,
    kernel_models/flash_attn.py:259).  s = q.k * (1/sqrt(D)); Mi = max_j s;
    Li = sum_j exp(s - Mi); O = sum_j exp(s - Mi) v_j / Li.  Computed in
    ``acc`` precision (fp64 by default) from whatever values Q/K/V hold.
    With ``causal`` / ``kv_lens`` only the keys of key_limits() enter each
    row, and with ``key_valid`` (bool [B, kv_len]) only valid keys; a row
    that sees none gets O = 0, Mi = -inf, Li = 0.
    """
    B, H_q, H_kv, q_len, kv_len, D = _check_shapes(Q, K, V)
    ratio = H_q // H_kv
    scale = acc(1.0) / np.sqrt(acc(D))
    masked = causal or kv_lens is not None or key_valid is not None
    lim = key_limits(q_len, kv_len, causal, kv_lens, B) if masked else None
    O = np.empty((B, H_q, q_len, D), dtype=acc)
    M = np.empty((B, H_q, q_len), dtype=acc)
    L = np.empty((B, H_q, q_len), dtype=acc)
    for b in range(B):
        for h in range(H_q):
            hk = h // ratio
            q = np.asarray(Q[b, h], dtype=acc)
            k = np.asarray(K[b, hk], dtype=acc)
            v = np.asarray(V[b, hk], dtype=acc)
            s = (q @ k.T) * scale
            if masked:
                visible = np.arange(kv_len)[None, :] < lim[b][:, None]
                if key_valid is not None:
                    visible = visible & np.asarray(key_valid[b], dtype=bool)[None, :]
                s = np.where(visible, s, -np.inf)
                empty = ~visible.any(axis=1)
                m = np.where(empty, 0.0, s.max(axis=1))
                p = np.exp(s - m[:, None])
                l = p.sum(axis=1)
                O[b, h] = (p @ v) / np.where(empty, 1.0, l)[:, None]
                M[b, h] = np.where(empty, -np.inf, m)
                L[b, h] = l
                continue
            m = s.max(axis=1)
            p = np.exp(s - m[:, None])
            l = p.sum(axis=1)
            O[b, h] = (p @ v) / l[:, None]
            M[b, h] = m
            L[b, h] = l
    return O, M, L


def sdpa_fp32_reference_style(Q, K, V):
    """fp32 SDPA in the exact operation order of kernel_models/flash_attn.py:250-265.

    Used as the timed CPU baseline (it is what the reference's NumPy path
    computes): per (b, h) one fp32 GEMM for the scores, max-subtract, exp,
    normalise, one fp32 GEMM with V.
    """
    B, H_q, H_kv, q_len, kv_len, D = _check_shapes(Q, K, V)
    ratio = H_q // H_kv
    scale = np.float32(1.0 / math.sqrt(float(D)))
    O = np.empty((B, H_q, q_len, D), dtype=np.float32)
    for b in range(B):
        for h in range(H_q):
            hk = h // ratio
            s = (Q[b, h].astype(np.float32) @ K[b, hk].astype(np.float32).T) * scale
            s -= s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            O[b, h] = p @ V[b, hk].astype(np.float32)
    return O


# ---------------------------------------------------------------------------
# Tiled online-softmax model (the reference's tile geometry)
# ---------------------------------------------------------------------------

def tiled_online_softmax(Q, K, V, br=16, bc_col=8, kv_block_rows=128):
    """Tiled flash-attention forward in fp32, prefill only (q_len == kv_len).

    Follows the loop structure of kernel_models/flash_attn.py:184-246 (query
    tiles of ``br`` rows; KV blocks of ``kv_block_rows``) and :87-180 (inside a
    block, key columns in tiles of ``bc_col``; per column tile: scores, mask,
    running max merge, exp, rescale of the running sum and output, P.V).  P is
    kept in fp32 as in the model (:166-167).  The 16-deep k loop and 8-wide
    co loop of the model are whole-row matmuls here; they are plain sums.
    Returns (O, Mi, Li) with Mi/Li in natural-log units of scaled scores.
    """
    B, H_q, H_kv, q_len, kv_len, D = _check_shapes(Q, K, V)
    if q_len != kv_len:
        raise ValueError("the tiled model is prefill-only (q_len == kv_len)")
    S = q_len
    ratio = H_q // H_kv
    scale = np.float32(1.0 / np.sqrt(np.float32(D)))
    O = np.zeros((B, H_q, S, D), dtype=np.float32)
    M = np.zeros((B, H_q, S), dtype=np.float32)
    L = np.zeros((B, H_q, S), dtype=np.float32)
    Qf = np.asarray(Q, dtype=np.float32)
    Kf = np.asarray(K, dtype=np.float32)
    Vf = np.asarray(V, dtype=np.float32)
    for b in range(B):
        for h in range(H_q):
            hk = h // ratio
            for q0 in range(0, S, br):
                q = Qf[b, h, q0:q0 + br]
                n_q = q.shape[0]
                m_run = np.full(n_q, -np.inf, dtype=np.float32)
                l_run = np.zeros(n_q, dtype=np.float32)
                o_run = np.zeros((n_q, D), dtype=np.float32)
                for k0 in range(0, S, kv_block_rows):
                    kb = Kf[b, hk, k0:k0 + kv_block_rows]
                    vb = Vf[b, hk, k0:k0 + kv_block_rows]
                    for c0 in range(0, kb.shape[0], bc_col):
                        kc = kb[c0:c0 + bc_col]
                        vc = vb[c0:c0 + bc_col]
                        s = (q @ kc.T) * scale
                        m_new = np.maximum(m_run, s.max(axis=1))
                        p = np.exp(s - m_new[:, None])
                        alpha = np.exp(m_run - m_new)
                        l_run = l_run * alpha + p.sum(axis=1)
                        o_run = o_run * alpha[:, None] + p @ vc
                        m_run = m_new
                O[b, h, q0:q0 + n_q] = o_run / l_run[:, None]
                M[b, h, q0:q0 + n_q] = m_run
                L[b, h, q0:q0 + n_q] = l_run
    return O, M, L


# ---------------------------------------------------------------------------
# Split-KV (flash-decoding) partials and merge
# ---------------------------------------------------------------------------

def split_bounds(kv_len: int, n_splits: int):
    """Contiguous, as-even-as-possible KV ranges [start, end) covering kv_len."""
    base, extra = divmod(kv_len, n_splits)
    out, start = [], 0
    for i in range(n_splits):
        n = base + (1 if i < extra else 0)
        out.append((start, start + n))
        start += n
    return out


def split_kv_partials(Q, K, V, bounds, acc=np.float64):
    """Per-split unnormalised partial states (O_k, m_k, l_k) over KV ranges.

    O_k = sum_{j in split} exp(s_j - m_k) v_j (unnormalised), m_k = max s_j,
    l_k = sum exp(s_j - m_k).  Empty ranges give m_k = -inf, l_k = 0, O_k = 0.
    """
    B, H_q, H_kv, q_len, kv_len, D = _check_shapes(Q, K, V)
    ratio = H_q // H_kv
    scale = acc(1.0) / np.sqrt(acc(D))
    n = len(bounds)
    Op = np.zeros((n, B, H_q, q_len, D), dtype=acc)
    Mp = np.full((n, B, H_q, q_len), -np.inf, dtype=acc)
    Lp = np.zeros((n, B, H_q, q_len), dtype=acc)
    for i, (s0, s1) in enumerate(bounds):
        if s1 <= s0:
            continue
        for b in range(B):
            for h in range(H_q):
                hk = h // ratio
                s = (np.asarray(Q[b, h], acc) @ np.asarray(K[b, hk, s0:s1], acc).T) * scale
                m = s.max(axis=1)
                p = np.exp(s - m[:, None])
                Op[i, b, h] = p @ np.asarray(V[b, hk, s0:s1], acc)
                Mp[i, b, h] = m
                Lp[i, b, h] = p.sum(axis=1)
    return Op, Mp, Lp


def split_kv_combine(Op, Mp, Lp):
    """Merge split partials: returns (O, Mi, Li) equal to sdpa's."""
    m = Mp.max(axis=0)
    w = np.where(np.isfinite(Mp), np.exp(Mp - m[None]), 0.0)
    l = (Lp * w).sum(axis=0)
    O = (Op * w[..., None]).sum(axis=0) / l[..., None]
    return O, m, l


# ---------------------------------------------------------------------------
# Metrics and tolerance
# ---------------------------------------------------------------------------

ATOL = 2e-3   # north_star: max-abs error
RTOL = 1e-2   # north_star: relative error, as ||got-ref||_2 / ||ref||_2


def errors(got, ref):
    """(max-abs error, relative L2 error) of ``got`` against ``ref``."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    diff = got - ref
    max_abs = float(np.abs(diff).max()) if diff.size else 0.0
    denom = float(np.linalg.norm(ref.ravel()))
    rel = float(np.linalg.norm(diff.ravel())) / denom if denom > 0 else float(np.linalg.norm(diff.ravel()))
    return max_abs, rel


def within_tolerance(got, ref, atol=ATOL, rtol=RTOL):
    max_abs, rel = errors(got, ref)
    return (max_abs <= atol and rel <= rtol), max_abs, rel


def attn_flops(B, H_q, q_len, kv_len, D):
    """4*B*H_q*q_len*kv_len*D (tests/bench_flash_attn.cu:125-126)."""
    return 4.0 * B * H_q * q_len * kv_len * D


def attn_bytes(B, H_q, H_kv, q_len, kv_len, D):
    """fp16 Q + unique fp16 K and V + fp32 O (tests/bench_flash_attn.cu:129-130)."""
    q_n = B * H_q * q_len * D
    kv_n = B * H_kv * kv_len * D
    return 2.0 * q_n + 2.0 * kv_n + 2.0 * kv_n + 4.0 * q_n
