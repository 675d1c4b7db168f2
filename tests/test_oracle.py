"""Pins for the CPU oracle (oracle/): published sequences, brute force, the
reference examples' known-answer patterns, and the committed golden vectors."""
import itertools
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layouts.json")
M64 = (1 << 64) - 1


def py_xorshift(seed, n):
    x, out = seed, []
    for _ in range(n):
        x ^= (x << 13) & M64
        x ^= x >> 7
        x ^= (x << 17) & M64
        out.append(x)
    return out


def test_xorshift_marsaglia_published_values():
    # Marsaglia, "Xorshift RNGs" (2003): x ^= x<<13; x ^= x>>7; x ^= x<<17 with
    # seed 88172645463325252 starts 8748534153485358512, 3040900993826735515,
    # 3453997556048239312.
    got = [int(v) for v in oracle.xorshift64_seq(88172645463325252, 3)]
    assert got == [8748534153485358512, 3040900993826735515, 3453997556048239312]


def test_xorshift_matches_python_for_benchmark_seeds():
    for seed in (oracle.DATA_SEED, oracle.PERM_SEED, oracle.LOGITS_SEED):
        assert [int(v) for v in oracle.xorshift64_seq(seed, 64)] == py_xorshift(seed, 64)


@pytest.mark.parametrize("t", [1, 5, 8, 12, 64, 4096])
def test_fill_tokens_is_the_byte_stream(t):
    n, stride = 7, 2 * t + 3
    region = np.zeros(n * stride, np.uint8)
    oracle.fill_tokens(region, n, t, stride, seed=oracle.DATA_SEED)
    words = py_xorshift(oracle.DATA_SEED, (n * t + 7) // 8 + 1)
    stream = b"".join(w.to_bytes(8, "little") for w in words)
    for k in range(n):
        tok = region[k * stride:k * stride + t].tobytes()
        assert tok == stream[k * t:(k + 1) * t]
        assert (region[k * stride + t:(k + 1) * stride] == oracle.GAP_BYTE).all()


def py_fisher_yates(n, seed):
    perm = list(range(n))
    xs = py_xorshift(seed, max(n - 1, 0))
    for step, i in enumerate(range(n - 1, 0, -1)):
        j = xs[step] % (i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    return perm


@pytest.mark.parametrize("n", [0, 1, 2, 3, 10, 257, 8192])
def test_permutation_is_a_bijection_and_matches_draw(n):
    p = oracle.permutation(n, seed=oracle.PERM_SEED)
    assert sorted(p.tolist()) == list(range(n))
    if n <= 257:
        assert p.tolist() == py_fisher_yates(n, oracle.PERM_SEED)


def test_permutation_uniform_over_all_orderings():
    # Brute force: every ordering of 4 items appears, roughly equally often.
    counts = {}
    for s in range(1, 4801):
        key = tuple(oracle.permutation(4, seed=s * 0x9E3779B97F4A7C15 & M64 or 1).tolist())
        counts[key] = counts.get(key, 0) + 1
    assert set(counts) == set(itertools.permutations(range(4)))
    assert min(counts.values()) > 100 and max(counts.values()) < 300  # expect 200 each


def naive_gather(region, perm, t, stride):
    out = bytearray()
    for j in perm:
        out += region[j * stride:j * stride + t].tobytes()
    return np.frombuffer(bytes(out), np.uint8)


@pytest.mark.parametrize("n,t", [(1, 16), (5, 7), (33, 100), (64, 4096)])
def test_expected_gather_matches_naive(n, t):
    stride = 2 * t
    region = np.empty(n * stride, np.uint8)
    oracle.fill_tokens(region, n, t, stride)
    perm = oracle.permutation(n)
    assert (oracle.expected_gather(region, perm, t, stride) == naive_gather(region, perm, t, stride)).all()


def naive_scatter(region, tokens, perm, t, stride):
    out = bytearray(region.tobytes())
    for j, p in enumerate(perm):
        for b in range(t):
            out[int(p) * stride + b] = int(tokens[j * t + b])
    return np.frombuffer(bytes(out), np.uint8)


@pytest.mark.parametrize("n,t,stride", [(1, 16, 16), (5, 7, 9), (33, 100, 200), (64, 64, 128)])
def test_expected_scatter_matches_naive(n, t, stride):
    rng = np.random.default_rng(n * 7 + t)
    region = rng.integers(0, 256, n * stride + 5, dtype=np.uint8)
    tokens = rng.integers(0, 256, n * t, dtype=np.uint8)
    perm = oracle.permutation(n)
    got = oracle.expected_scatter(region, tokens, perm, t, stride)
    assert (got == naive_scatter(region, tokens, perm, t, stride)).all()


@pytest.mark.parametrize("n,t", [(3, 1), (100, 48), (512, 4096)])
def test_expected_scatter_inverts_gather(n, t):
    """Offload then gather with the same order returns the tokens; bytes no
    token covers (the 2x-stride gaps) keep the sentinel."""
    rng = np.random.default_rng(n + t)
    stride = 2 * t
    tokens = rng.integers(0, 256, n * t, dtype=np.uint8)
    perm = oracle.permutation(n)
    region = np.full(n * stride, 0xCD, np.uint8)
    out = oracle.expected_scatter(region, tokens, perm, t, stride)
    assert (oracle.expected_gather(out, perm, t, stride) == tokens).all()
    assert (out.reshape(n, 2, t)[:, 1, :] == 0xCD).all()
    # The inverse order in place of the order (a transposed index) is caught
    # whenever the order is not its own inverse.
    inv = np.argsort(perm).astype(np.uint32)
    if not (inv == perm).all():
        wrong = oracle.expected_scatter(region, tokens, inv, t, stride)
        assert not (oracle.expected_gather(wrong, perm, t, stride) == tokens).all()


def test_gather_entries_closed_form_with_gaps():
    rng = np.random.default_rng(1)
    src = rng.integers(0, 256, 50000, dtype=np.uint8)
    sizes = [1, 63, 64, 65, 200, 4096, 3]
    entries = (oracle.SGEntry * len(sizes))()
    dst, s_off, expect = 0, 0, np.zeros(6000, np.uint8)
    for i, sz in enumerate(sizes):
        entries[i].dst = 1000 + dst
        entries[i].src = src.ctypes.data + s_off
        entries[i].size = sz
        expect[dst:dst + sz] = src[s_off:s_off + sz]
        dst += sz + 5  # leave gaps
        s_off += 3 * sz + 1
    out = oracle.gather_entries(entries, len(sizes), 6000, 1000)
    assert (out == expect).all()


@pytest.mark.parametrize("workers", [0, 1, 3, 7, 15])
@pytest.mark.parametrize("n,t", [(1, 4096), (3, 4096), (256, 4096), (100, 1000), (40, 65536), (17, 70)])
def test_pool_gather_equals_closed_form(workers, n, t):
    # src/parallel_gather.cpp:74-116 restated; result independent of W and of
    # the 64-byte body / memcpy tail split.
    stride = 2 * t
    region = np.empty(n * stride, np.uint8)
    oracle.fill_tokens(region, n, t, stride)
    perm = oracle.permutation(n)
    base = 1 << 40
    entries = oracle.make_entries(region.ctypes.data, base, perm, t, stride)
    staging = np.zeros(n * t + 64, np.uint8)
    staging[n * t:] = 0x5A
    pool = oracle.GatherPool(workers)
    try:
        pool.gather(entries, n, staging, base)
    finally:
        pool.close()
    assert (staging[:n * t] == oracle.expected_gather(region, perm, t, stride)).all()
    assert (staging[n * t:] == 0x5A).all()  # nothing written past the range


def test_reference_kat_direct_transfer_pattern():
    # examples/02_direct_transfer.cu:50-54,117-129: 1024 tokens x 4 KB at 2x
    # stride, token i = memset(i & 0xFF), gathered in order, full byte compare.
    n, t, stride = 1024, 4096, 8192
    region = np.full(n * stride, oracle.GAP_BYTE, np.uint8)
    for i in range(n):
        region[i * stride:i * stride + t] = i & 0xFF
    perm = np.arange(n, dtype=np.uint32)
    entries = oracle.make_entries(region.ctypes.data, 0, perm, t, stride)
    staging = np.zeros(n * t, np.uint8)
    pool = oracle.GatherPool(3)
    try:
        pool.gather(entries, n, staging, 0)
    finally:
        pool.close()
    expect = np.repeat((np.arange(n) & 0xFF).astype(np.uint8), t)
    assert (staging == expect).all()
    gold = json.load(open(GOLDEN))["kat_direct_transfer"]
    assert "%016x" % oracle.fnv1a64(staging) == gold["output_fnv1a64"]


def test_reference_kat_float_patterns():
    # examples/01_basic_transfer.cu:138-142 (float t*1000+d) and
    # test/test_sg_e2e.cu:42 (float i+1): the gather moves the float bit
    # patterns unchanged.
    n, dim = 16, 1024
    t = dim * 4
    vals = (np.arange(n)[:, None] * 1000 + np.arange(dim)[None, :]).astype(np.float32)
    region = np.full(n * 2 * t, oracle.GAP_BYTE, np.uint8)
    for i in range(n):
        region[i * 2 * t:i * 2 * t + t] = vals[i].view(np.uint8)
    perm = oracle.permutation(n)
    out = oracle.expected_gather(region, perm, t, 2 * t).view(np.float32).reshape(n, dim)
    assert (out == vals[perm]).all()
    ones = (np.arange(4 * 1024) + 1).astype(np.float32)
    out2 = oracle.expected_gather(ones.view(np.uint8), np.arange(4, dtype=np.uint32), 4096, 4096)
    assert (out2.view(np.float32) == ones).all()


def test_fnv1a64_published_vectors():
    # FNV-1a 64-bit test vectors (Fowler/Noll/Vo reference table).
    assert oracle.fnv1a64(np.frombuffer(b"", np.uint8)) == 0xCBF29CE484222325
    assert oracle.fnv1a64(np.frombuffer(b"a", np.uint8)) == 0xAF63DC4C8601EC8C
    assert oracle.fnv1a64(np.frombuffer(b"foobar", np.uint8)) == 0x85944171F73967E8


def test_golden_layouts():
    gold = json.load(open(GOLDEN))
    assert gold["seeds"]["data"] == "%016x" % oracle.DATA_SEED
    for name, seed in (("data", oracle.DATA_SEED), ("perm", oracle.PERM_SEED), ("logits", oracle.LOGITS_SEED)):
        assert gold["xorshift_head"][name] == ["%016x" % x for x in py_xorshift(seed, 8)]
    for name, g in gold["layouts"].items():
        n, t, stride = g["num_tokens"], g["token_size"], g["stride"]
        region = np.empty(n * stride, np.uint8)
        oracle.fill_tokens(region, n, t, stride)
        perm = oracle.permutation(n)
        assert perm[:32].tolist() == g["perm_head"], name
        assert "%016x" % oracle.fnv1a64(perm) == g["perm_fnv1a64"], name
        assert "%016x" % oracle.fnv1a64(region) == g["region_fnv1a64"], name
        out = oracle.expected_gather(region, perm, t, stride)
        assert "%016x" % oracle.fnv1a64(out) == g["output_fnv1a64"], name


# ------------------------------------------------------------------ MoE (C5)

def test_moe_logits_formula_and_range():
    lg = oracle.moe_logits(8, 64)
    xs = py_xorshift(oracle.LOGITS_SEED, 8 * 64)
    expect = np.array([((x >> 40) / float(1 << 24)) * 8.0 - 4.0 for x in xs], np.float32).reshape(8, 64)
    assert (lg == expect).all()
    big = oracle.moe_logits(4096, 64)
    assert big.min() >= -4.0 and big.max() < 4.0


def test_moe_top2_brute_force_and_ties():
    lg = oracle.moe_logits(200, 16)
    top = oracle.moe_top2(lg)
    for t in range(200):
        order = sorted(range(16), key=lambda e: (-float(lg[t, e]), e))
        assert top[t].tolist() == order[:2]
    tie = np.zeros((1, 8), np.float32)
    tie[0, [6, 2, 5]] = 1.0
    assert oracle.moe_top2(tie)[0].tolist() == [2, 5]  # ties -> lower expert id
    # top-2 of softmax == top-2 of logits (softmax is monotone)
    sm = np.exp(lg - lg.max(1, keepdims=True))
    sm /= sm.sum(1, keepdims=True)
    assert (np.sort(oracle.moe_top2(lg), 1) == np.sort(np.argsort(-sm, 1, kind="stable")[:, :2], 1)).all()


def test_moe_lists_stable_and_complete():
    lg = oracle.moe_logits(512, 64)
    top = oracle.moe_top2(lg)
    offsets, rows = oracle.moe_lists(top, 64)
    assert offsets[-1] == 2 * 512
    for e in range(64):
        seg = rows[offsets[e]:offsets[e + 1]]
        assert (np.diff(seg) > 0).all()  # token order, each token once per expert
        assert set(seg.tolist()) == set(np.nonzero((top == e).any(1))[0].tolist())
    gold = json.load(open(GOLDEN))["moe_4096x64"]
    lg = oracle.moe_logits(4096, 64)
    offsets, rows = oracle.moe_lists(oracle.moe_top2(lg), 64)
    assert np.diff(offsets).tolist() == gold["expert_counts"]
    assert "%016x" % oracle.fnv1a64(rows.astype(np.int32)) == gold["rows_fnv1a64"]


def test_rmsnorm_closed_forms():
    x = np.full((3, 128), 2.0, np.float32)
    w = np.ones(128, np.float32)
    y = oracle.rmsnorm_rows(x, w, 0.0)
    assert np.allclose(y, 1.0)  # constant row c: c / |c| = 1
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    w = np.ones(256, np.float32)
    y1 = oracle.rmsnorm_rows(x, w, 0.0)
    y2 = oracle.rmsnorm_rows(7.5 * x, w, 0.0)
    assert np.allclose(y1, y2, atol=1e-5)  # scale invariance at eps = 0
    assert np.allclose(np.mean(y1.astype(np.float64) ** 2, 1), 1.0, atol=1e-5)
    w2 = rng.standard_normal(256).astype(np.float32)
    assert np.allclose(oracle.rmsnorm_rows(x, w2, 0.0), y1 * w2, atol=1e-5)


@pytest.mark.timeout(120)
def test_pool_back_to_back_gathers_do_not_lose_tasks():
    # Regression for the task hand-off order: thousands of back-to-back
    # gathers must all complete (a worker that clears has_work after raising
    # done can erase the next task and stall the caller).
    n, t = 64, 4096
    region = np.empty(n * 2 * t, np.uint8)
    oracle.fill_tokens(region, n, t, 2 * t)
    perm = oracle.permutation(n)
    entries = oracle.make_entries(region.ctypes.data, 0, perm, t, 2 * t)
    staging = np.zeros(n * t, np.uint8)
    pool = oracle.GatherPool(7)
    try:
        times = pool.time(entries, n, staging, 0, 3000)
    finally:
        pool.close()
    assert len(times) == 3000
    assert (staging == oracle.expected_gather(region, perm, t, 2 * t)).all()


def test_bf16_rounding_known_values():
    # Round-to-nearest-even: 1 + 2^-8 is halfway between bf16 1.0 and
    # 1 + 2^-7 and goes to the even one; 1 + 3*2^-9 rounds up; the result of
    # every representable bf16 value is itself.
    x = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -9, -2.5, 0.0], np.float32)
    assert oracle.f32_to_bf16(x).tolist() == [0x3F80, 0x3F80, 0x3F81, 0xC020, 0x0000]
    allb = np.arange(0, 0x7F80, 7, dtype=np.uint16)
    assert (oracle.f32_to_bf16(oracle.bf16_to_f32(allb)) == allb).all()


def test_moe_token_values_and_weight_ranges():
    v = oracle.bf16_to_f32(oracle.moe_token_values(16, 512))
    assert v.min() >= -1.0 and v.max() <= 1.0 and np.isfinite(v).all()
    w = oracle.bf16_to_f32(oracle.moe_weight(512))
    assert w.min() >= 0.5 and w.max() <= 1.5


# ------------------------------------------------------------ sessions

@pytest.mark.parametrize("token_size,db,expect", [
    # ~128 KiB chunks: 4 KiB tokens -> 32 per chunk, 4 chunks per 128-token tile
    (4096, False, (32, 4, 64 * 5)),
    # small tokens aim at 64 KiB: 512 B -> 128 tokens = the whole tile
    (512, False, (128, 1, 128)),
    (256, False, (128, 1, 128)),
    (1024, False, (128, 1, 128)),
    (2048, False, (64, 2, 64 * 3)),
    # 16 KiB tokens: 8 per chunk would be 16 chunks; the K <= 8 limit raises it to 16
    (16384, False, (16, 8, 64 * 9)),
    # large tokens aim at 256 KiB: 4 tokens, again raised to the K <= 8 floor
    (65536, False, (16, 8, 64 * 9)),
    # double buffering: K <= 4 keeps 1 + 2K waves within 1024 threads
    (16384, True, (32, 4, 64 * 9)),
    (4096, True, (32, 4, 64 * 9)),
    (3000, False, (32, 4, 64 * 5)),   # 131072 // 3000 = 43 -> 32
])
def test_warp_spec_chunking_known(token_size, db, expect):
    assert oracle.warp_spec_chunking(token_size, 128, 0, db) == expect


def test_warp_spec_chunking_explicit_and_per_tile():
    # test/test_db_small_tiles.cu: tile 32 / chunk 16 (K=2), 16/16 (K=1), 64/16 (K=4), double-buffered
    assert oracle.warp_spec_chunking(1024, 32, 16, True) == (16, 2, 64 * 5)
    assert oracle.warp_spec_chunking(1024, 16, 16, True) == (16, 1, 64 * 3)
    assert oracle.warp_spec_chunking(1024, 64, 16, True) == (16, 4, 64 * 9)
    assert oracle.warp_spec_chunking(4096, 128, 0, False, per_tile_mode=True) == (128, 1, 128)


def test_warp_spec_chunking_invariants():
    for T in (16, 32, 64, 128, 256, 512):
        for ts in (16, 100, 512, 513, 4096, 5000, 65535, 65536, 1 << 20):
            for db in (False, True):
                c, k, block = oracle.warp_spec_chunking(ts, T, 0, db)
                assert c & (c - 1) == 0 and T % c == 0 and k * c == T
                assert k <= (4 if db else 8) and block <= 1024
                target = 65536 if ts <= 512 else (262144 if ts >= 65536 else 131072)
                raw = max(4, target // ts)
                if T // (4 if db else 8) <= raw <= T:
                    # unclamped: the largest power of two not above the target
                    assert c <= raw < 2 * c


def test_warp_spec_expected_brute_force():
    rng = np.random.default_rng(5)
    for total, ts, T in [(10, 3, 4), (8, 5, 8), (7, 2, 8), (33, 16, 16)]:
        src = rng.integers(0, 256, total * ts, dtype=np.uint8)
        before = rng.integers(0, 256, total * ts, dtype=np.uint8)
        want = before.copy()
        for t in range((total // T) * T):
            for b in range(ts):
                want[t * ts + b] = src[t * ts + b]
        assert (oracle.warp_spec_expected(src, before, total, ts, T) == want).all()


def test_u32_word_checksum():
    # closed forms
    for n in (0, 1, 3, 4, 5, 64, 1027):
        assert oracle.u32_word_checksum(np.ones(n, np.uint8)) == (n // 4) * 0x01010101 + n % 4
    assert oracle.u32_word_checksum(np.array([0x78, 0x56, 0x34, 0x12], np.uint8)) == 0x12345678
    # independent little-endian loop
    rng = np.random.default_rng(9)
    for n in (1, 7, 64, 255):
        b = rng.integers(0, 256, n, dtype=np.uint8)
        ref = sum(int.from_bytes(bytes(b[i:i + 4]), "little") for i in range(0, n - n % 4, 4))
        ref += sum(int(x) for x in b[n - n % 4:])
        assert oracle.u32_word_checksum(b) == ref
