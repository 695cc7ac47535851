"""GPU parity at the edges of every tiling boundary of the kernels, which
random shapes rarely hit exactly: key counts around the 32-key MFMA tile,
the 64-key prefill stage and the 256-key minimum split of the 8-wave
streaming decode; query rows per KV head around 32 (the decode / prefill
switch) and around the 32 / 64 / 256-row workgroup tiles; causal masks with
more queries than keys (rows that see no key) and per-sequence key counts
at 0, 1 and full.  Each case is checked against the fp64 oracle at the
north-star bar (tests/_parity.py)."""
import pytest

from tests._parity import run_and_check

pytestmark = pytest.mark.gpu


def _cases():
    out = []
    seed = 500
    # Decode (R <= 32): key counts around tile, split and stage edges.
    for kv in (31, 32, 33, 63, 64, 65, 255, 256, 257, 511, 512, 513):
        for (H_q, H_kv, D) in ((32, 8, 128), (32, 1, 64)):
            seed += 1
            out.append((2, H_q, H_kv, 1, kv, D, False, None, seed))
    # Streaming decode (large batch) at its split edges, with key counts.
    for kv in (255, 256, 257, 2047, 2048, 2049):
        seed += 1
        out.append((12, 8, 8, 1, kv, 128, False, [kv, kv - 1, 1, 0] * 3, seed))
    # Rows per KV head around 32: 8 x 4 = 32 (decode), 9 x 4 = 36 (prefill).
    for q in (7, 8, 9):
        seed += 1
        out.append((1, 8, 2, q, 300, 128, True, None, seed))
    # Prefill row / key counts around tile, stage and workgroup edges.
    for (q, kv) in ((31, 33), (32, 32), (33, 31), (63, 65), (64, 64), (65, 63),
                    (255, 257), (256, 256), (257, 255)):
        for D in (64, 128):
            seed += 1
            out.append((1, 4, 1, q, kv, D, seed % 2 == 0, None, seed))
    # Causal with more queries than keys: the first q - kv rows see no key.
    for (q, kv, D) in ((100, 40, 128), (70, 1, 64), (300, 257, 256)):
        seed += 1
        out.append((1, 4, 2, q, kv, D, True, None, seed))
    # Per-sequence key counts at 0, 1 and full on the prefill path.
    seed += 1
    out.append((3, 8, 2, 96, 160, 128, False, [0, 1, 160], seed))
    seed += 1
    out.append((3, 8, 2, 96, 160, 64, True, [160, 0, 1], seed))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_q{}_kv{}_D{}_c{}_{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], int(c[6]), "lens" if c[7] is not None else "full"))
def test_boundary_shape_parity(case):
    run_and_check(*case)
