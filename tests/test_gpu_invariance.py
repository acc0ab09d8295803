"""Invariances and concurrency the reference's own tests hold.

- A prefill split in two at S/2 gives the attention of one whole prefill,
  and decoding the token at position p over the cache a prefill left gives
  what a prefill of that token gives: the cache is an optimisation and must
  not change the numbers (src/llm-testing.cpp:576-613, which holds logits to
  5e-3). The reference's cache is fp32; this one is bf16, so a path that
  reads keys back from the cache sees them rounded where a single pass keeps
  them as computed, and each side is also held to the oracle of what it
  reads.
- Concurrent host-form callers do not overwrite each other's staged inputs
  or outputs, and every call is counted (src/gpu-testing.cpp:190-226: four
  threads of three repeats each)."""
import threading

import numpy as np
import pytest

from common import assert_bf16_parity, assert_f32_parity, bf16_normal, gammas
from gpu_util import dev_bf16, dev_f32, dev_u32, host, host_bits, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def inputs(S, H, KV, D, seed):
    qb, q = bf16_normal((S, H, D), seed, "q")
    kb, k = bf16_normal((S, KV, D), seed, "k")
    vb, v = bf16_normal((S, KV, D), seed, "v")
    return (qb, kb, vb), (q, k, v), gammas(D, seed, "q_norm"), gammas(D, seed, "k_norm"), \
        O.rotary_frequencies(D, 1e6)


def oracle_prefill(q, k, v, gq, gk, fr, S, H, KV, D, window, split=None):
    """attention over [0, S) in one pass; with `split`, rows from `split` on
    see the keys before it as the bf16 cache holds them"""
    qn, kn = O.qk_norm_rope(q, k, S, 0, H, KV, D, D, gq, gk, 1e-6, fr, D)
    whole = O.attention_strided(qn, kn, v, S, 0, H, KV, D, D, KV * D, D, window, nthreads=0)
    if split is None:
        return whole
    keys = np.concatenate([O.round_bf16(kn[:split]), kn[split:]], 0)
    second = O.attention_strided(np.ascontiguousarray(qn[split:]), keys, v, S - split, split, H, KV, D, D, KV * D,
                                 D, window, nthreads=0)
    return np.concatenate([whole[:split], second], 0)


def run_prefill(gpu, bits, rows, start, cache, H, KV, D, gq, gk, fr, window):
    import torch
    qb, kb, vb = bits
    a, b = rows
    out = torch.zeros((b - a, H, D), dtype=torch.float32, device="cuda")
    say("prefill rows", dict(a=a, b=b, start=start, H=H, KV=KV, D=D, window=window))
    gpu.prefill(dev_bf16(qb[a:b]), dev_bf16(kb[a:b]), dev_bf16(vb[a:b]), out, cache[0], cache[1], start, H, KV,
                D, q_norm=dev_f32(gq), k_norm=dev_f32(gk), freqs=dev_f32(fr), rotary_dims=D, window=window)
    return host(out)


def empty_cache(KV, cap, D):
    import torch
    return (torch.zeros((KV, cap, D), dtype=torch.bfloat16, device="cuda"),
            torch.zeros((KV, cap, D), dtype=torch.bfloat16, device="cuda"))


@pytest.mark.parametrize("S,window", [(300, 0), (300, 37), (1030, 0)])
def test_split_prefill_matches_whole(gpu, S, window):
    """positions [0, S/2) then [S/2, S) against [0, S) in one call. The second
    half of a split reads the first half's keys back from the bf16 cache
    while the whole call keeps them as computed (in fp16), so the two agree
    to the reference's own bar for this check, 5e-3 (llm-testing.cpp:
    598-610), each within the bf16 bar of the oracle, not bit for bit; the
    caches they leave are identical."""
    H, KV, D = 8, 2, 128
    bits, (q, k, v), gq, gk, fr = inputs(S, H, KV, D, 21)
    half = S // 2
    ref = oracle_prefill(q, k, v, gq, gk, fr, S, H, KV, D, window)
    ref_split = oracle_prefill(q, k, v, gq, gk, fr, S, H, KV, D, window, split=half)
    whole_cache, split_cache = empty_cache(KV, S, D), empty_cache(KV, S, D)
    whole = run_prefill(gpu, bits, (0, S), 0, whole_cache, H, KV, D, gq, gk, fr, window)
    first = run_prefill(gpu, bits, (0, half), 0, split_cache, H, KV, D, gq, gk, fr, window)
    second = run_prefill(gpu, bits, (half, S), half, split_cache, H, KV, D, gq, gk, fr, window)
    split = np.concatenate([first, second], 0)
    assert_bf16_parity(ref, whole, "whole")
    assert_bf16_parity(ref_split, split, "split")
    assert np.abs(whole - split).max() < 5e-3, "split against whole"
    # the first half sees the same keys, the same way, in both
    assert np.abs(first - whole[:half]).max() <= 1e-6
    for a, b in zip(whole_cache, split_cache):
        assert np.array_equal(host_bits(a), host_bits(b)), "caches differ"


@pytest.mark.parametrize("p", [0, 1, 77, 255, 256, 399])
def test_decode_at_p_matches_prefill_row_p(gpu, p):
    """the cache rows [0, p) written by a prefill of the first p tokens; then
    the token at position p both decoded and prefilled (count 1, start p)
    over copies of that cache. The two agree to the bf16 bar, each is within
    it of the oracle over the same cache (the history keys as bf16 holds
    them), and both append the same row p."""
    import torch
    S, H, KV, D = 400, 16, 8, 128
    bits, (q, k, v), gq, gk, fr = inputs(S, H, KV, D, 22)
    qb, kb, vb = bits
    cache = empty_cache(KV, S, D)
    if p:
        run_prefill(gpu, bits, (0, p), 0, cache, H, KV, D, gq, gk, fr, 0)
    kbits, vbits = host_bits(cache[0]), host_bits(cache[1])
    pcache = (dev_bf16(kbits), dev_bf16(vbits))
    pre = run_prefill(gpu, bits, (p, p + 1), p, pcache, H, KV, D, gq, gk, fr, 0)[0]
    dkc, dvc = dev_bf16(kbits), dev_bf16(vbits)
    out = torch.zeros((1, H, D), dtype=torch.float32, device="cuda")
    say("decode at p", dict(p=p, S=S, H=H, KV=KV, D=D))
    gpu.decode(dev_bf16(qb[p:p + 1]), dev_bf16(kb[p:p + 1]), dev_bf16(vb[p:p + 1]), out, dkc, dvc,
               dev_u32(np.array([p], np.uint32)), p, H, KV, D, q_norm=dev_f32(gq), k_norm=dev_f32(gk),
               freqs=dev_f32(fr), rotary_dims=D)
    got = host(out)[0]
    ref = oracle_prefill(q[:p + 1], k[:p + 1], v[:p + 1], gq, gk, fr, p + 1, H, KV, D, 0, split=p)[p]
    assert_bf16_parity(ref, pre, f"prefill at {p}")
    assert_bf16_parity(ref, got, f"decode at {p}")
    assert_bf16_parity(pre, got, f"decode against prefill at {p}")
    pk, pv = host_bits(pcache[0]), host_bits(pcache[1])
    dk, dv = host_bits(dkc), host_bits(dvc)
    assert np.array_equal(dv[:, p], pv[:, p]), "appended value"
    # the new key is normed and rotated by each path's own code: one bf16 ulp
    diff = np.abs(dk[:, p].astype(np.int32) - pk[:, p].astype(np.int32))
    assert diff.max() <= 1, f"appended key differs by {diff.max()} bf16 ulps"
    assert np.array_equal(dk[:, :p], kbits[:, :p]) and not dk[:, p + 1:].any()


def test_concurrent_host_calls(gpu):
    """four threads, each three times host-form aigpu_matmul_nt and
    aigpu_attention on inputs of its own size, into outputs of its own; the
    results equal the oracle's and the launch counter grows by exactly what
    the same calls add when made one at a time"""
    K, N, count, repeats = 96, 37, 4, 3
    w = O.fill_normal((N, K), 31, "w")
    wptr = gpu.upload(w)
    try:
        a = [O.fill_normal((i + 1, K), 31, f"a{i}") for i in range(count)]
        mm_ref = [O.matmul_nt(x, w, "f32") for x in a]
        shapes = [(3 + 5 * i, 2 * i, 4, 2, 64) for i in range(count)]   # count, start, H, KV, D
        att_in, att_ref = [], []
        for i, (T, S, H, KV, D) in enumerate(shapes):
            q = O.fill_normal((T, H, D), 32, f"q{i}")
            kk = O.fill_normal((S + T, KV, D), 32, f"k{i}")
            vv = O.fill_normal((S + T, KV, D), 32, f"v{i}")
            att_in.append((q, kk, vv))
            att_ref.append(O.attention(q, kk, vv, T, S, H, KV, D, D))

        def one(i):
            c = gpu.matmul_host(a[i], wptr, "f32", N)
            T, S, H, KV, D = shapes[i]
            o = gpu.attention(*att_in[i], T, S, H, KV, D, D)
            return c, o

        # what one round of calls adds to the counter, one caller at a time
        gpu.lib().aigpu_reset_counters()
        for i in range(count):
            c, o = one(i)
            assert_f32_parity(mm_ref[i], c, f"matmul {i}")
            assert_f32_parity(att_ref[i], o, f"attention {i}")
        per_round = gpu.counters()["launches"]
        assert per_round >= 2 * count

        gpu.lib().aigpu_reset_counters()
        results = [[None] * repeats for _ in range(count)]
        errors = []

        def worker(i):
            try:
                for r in range(repeats):
                    results[i][r] = one(i)
            except Exception as e:   # reported by the main thread
                errors.append(e)

        say("concurrent host calls", dict(threads=count, repeats=repeats))
        threads = [threading.Thread(target=worker, args=(i,)) for i in range(count)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert not errors, errors
        for i in range(count):
            for r in range(repeats):
                c, o = results[i][r]
                assert_f32_parity(mm_ref[i], c, f"matmul thread {i} repeat {r}")
                assert_f32_parity(att_ref[i], o, f"attention thread {i} repeat {r}")
        assert gpu.counters()["launches"] == repeats * per_round
    finally:
        gpu.release(wptr, w.nbytes)


def test_calls_on_two_streams_keep_their_scratch_apart(gpu):
    """device-form decodes issued back to back on two streams, with no
    synchronisation between them, share the backend's split-K record scratch;
    each call waits for the other stream's previous call, so both give what
    the same calls give one after another on one stream (bit for bit)"""
    import torch
    B, H, KV, D, L = 16, 32, 4, 128, 9000
    gen = torch.Generator(device="cuda").manual_seed(41)

    def case():
        q = torch.randn((B, H, D), generator=gen, device="cuda").to(torch.bfloat16)
        k = torch.randn((B, KV, D), generator=gen, device="cuda").to(torch.bfloat16)
        v = torch.randn((B, KV, D), generator=gen, device="cuda").to(torch.bfloat16)
        kc = torch.randn((B, KV, L + 1, D), generator=gen, device="cuda").to(torch.bfloat16)
        vc = torch.randn((B, KV, L + 1, D), generator=gen, device="cuda").to(torch.bfloat16)
        pos = torch.full((B,), L, dtype=torch.int32, device="cuda")
        return q, k, v, kc, vc, pos

    cases = [case(), case()]

    def run(c, caches, out, stream=None):
        q, k, v, _, _, pos = c
        gpu.decode(q, k, v, out, caches[0], caches[1], pos, L, H, KV, D,
                   stream=None if stream is None else stream.cuda_stream)

    def fresh_caches():
        return [(c[3].clone(), c[4].clone()) for c in cases]

    ref = [torch.zeros((B, H, D), device="cuda") for _ in cases]
    for c, cc, o in zip(cases, fresh_caches(), ref):
        run(c, cc, o)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    say("decode on two streams", dict(B=B, L=L))
    for rep in range(3):
        got = [torch.zeros((B, H, D), device="cuda") for _ in cases]
        caches = fresh_caches()
        torch.cuda.synchronize()   # inputs ready before either stream starts
        run(cases[0], caches[0], got[0], s1)
        run(cases[1], caches[1], got[1], s2)
        torch.cuda.synchronize()
        for g, r in zip(got, ref):
            assert torch.equal(g, r), f"repeat {rep}: a call's records were overwritten"
