"""aigpu_decode_attention_static, the decode entry point that allocates
nothing, against aigpu_decode_attention through the C ABI: the same kernels on
the same inputs, so outputs and appended cache rows must be bit-identical.
Two calls in a row, the second smaller, then a call whose one sequence needs
more split-K records than the fixed scratch holds, which must be refused
before any launch."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import dev_bf16, dev_f32, dev_u32, host, host_bits, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _args(aigpu, q, k, v, out, kc, vc, pos, max_pos, H, KV, D, qn, kn, fr, stream=None):
    return aigpu.AiGpuDecode(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), out=out.data_ptr(), keyCache=kc.data_ptr(),
        valueCache=vc.data_ptr(), positions=pos.data_ptr(), qNorm=qn.data_ptr(), kNorm=kn.data_ptr(),
        rotaryFrequencies=fr.data_ptr(), epsilon=1e-6, normOffset=0.0, rotaryDims=D, inType=1,
        maxPosition=max_pos, outputGate=0, batch=q.shape[0], heads=H, kvHeads=KV, dim=D, qStride=D, window=0,
        capacity=kc.shape[-2], batchStride=0, stream=stream)


def _case(gpu, B, H, KV, D, lengths, seed):
    import torch
    cap = max(lengths) + 1
    qb = O.pack_bf16(O.fill_normal((B, H, D), seed, "q"))
    kb = O.pack_bf16(O.fill_normal((B, KV, D), seed, "k"))
    vb = O.pack_bf16(O.fill_normal((B, KV, D), seed, "v"))
    hist = O.pack_bf16(O.fill_normal((B, KV, cap, D), seed, "cache"))
    q, k, v = dev_bf16(qb), dev_bf16(kb), dev_bf16(vb)
    qn = dev_f32(O.fill_uniform((D,), seed, "gq", 0.5, 1.5))
    kn = dev_f32(O.fill_uniform((D,), seed, "gk", 0.5, 1.5))
    fr = dev_f32(O.rotary_frequencies(D, 1e6))
    pos = dev_u32(np.array(lengths, np.uint32))
    results = []
    for name in ("aigpu_decode_attention", "aigpu_decode_attention_static"):
        kc, vc = dev_bf16(hist), dev_bf16(hist[:, :, ::-1].copy())
        out = torch.zeros((B, H, D), dtype=torch.float32, device="cuda")
        a = _args(gpu, q, k, v, out, kc, vc, pos, max(lengths), H, KV, D, qn, kn, fr)
        say(name, dict(B=B, H=H, KV=KV, D=D, max_len=max(lengths)))
        rc = getattr(gpu.lib(), name)(C.byref(a))
        assert rc == 1, gpu.last_error()
        results.append((host(out), host_bits(kc), host_bits(vc)))
    (o0, k0, v0), (o1, k1, v1) = results
    assert np.array_equal(o0, o1), f"max diff {np.abs(o0 - o1).max()}"
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    assert np.isfinite(o1).all() and np.abs(o1).max() > 0


def test_static_decode_matches_the_allocating_entry_point(gpu):
    r = np.random.default_rng(7)
    _case(gpu, 32, 32, 4, 128, [int(x) for x in r.integers(1000, 9000, 32)], 21)
    # second call with a smaller input, reusing the same fixed scratch
    _case(gpu, 3, 16, 8, 128, [700, 33, 4096], 22)


def test_static_decode_replays_from_a_captured_graph(gpu):
    """the entry point is for callers that cannot allocate, such as code under
    graph capture: one eager call first (it sets up the backend and looks up
    the fixed scratch's address), then the call captured into a torch CUDA
    graph and replayed three times, with eager decodes of other sizes and
    synchronisations between the replays; every replay's output and appended
    cache rows equal the eager call's bit for bit"""
    import torch
    B, H, KV, D, lengths, seed = 5, 16, 4, 128, [4100, 17, 2900, 9000, 640], 23
    cap = max(lengths) + 1
    qb = O.pack_bf16(O.fill_normal((B, H, D), seed, "q"))
    kb = O.pack_bf16(O.fill_normal((B, KV, D), seed, "k"))
    vb = O.pack_bf16(O.fill_normal((B, KV, D), seed, "v"))
    hist = O.pack_bf16(O.fill_normal((B, KV, cap, D), seed, "cache"))
    q, k, v = dev_bf16(qb), dev_bf16(kb), dev_bf16(vb)
    qn = dev_f32(O.fill_uniform((D,), seed, "gq", 0.5, 1.5))
    kn = dev_f32(O.fill_uniform((D,), seed, "gk", 0.5, 1.5))
    fr = dev_f32(O.rotary_frequencies(D, 1e6))
    pos = dev_u32(np.array(lengths, np.uint32))

    def fresh():
        return (dev_bf16(hist), dev_bf16(hist[:, :, ::-1].copy()),
                torch.zeros((B, H, D), dtype=torch.float32, device="cuda"))

    kc, vc, out = fresh()
    say("aigpu_decode_attention_static eager", dict(B=B, H=H, KV=KV, D=D, max_len=max(lengths)))
    assert gpu.lib().aigpu_decode_attention_static(
        C.byref(_args(gpu, q, k, v, out, kc, vc, pos, max(lengths), H, KV, D, qn, kn, fr))) == 1, gpu.last_error()
    want = (host(out), host_bits(kc), host_bits(vc))

    kc, vc, out = fresh()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    say("aigpu_decode_attention_static capture", dict(B=B))
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            a = _args(gpu, q, k, v, out, kc, vc, pos, max(lengths), H, KV, D, qn, kn, fr,
                      stream=side.cuda_stream)
            rc = gpu.lib().aigpu_decode_attention_static(C.byref(a))
    torch.cuda.current_stream().wait_stream(side)
    assert rc == 1, gpu.last_error()
    for replay in range(3):
        out.zero_()
        say("aigpu_decode_attention_static replay", dict(replay=replay))
        graph.replay()
        torch.cuda.synchronize()
        got = (host(out), host_bits(kc), host_bits(vc))
        assert np.array_equal(got[0], want[0]), f"replay {replay}: max diff {np.abs(got[0] - want[0]).max()}"
        assert np.array_equal(got[1], want[1]) and np.array_equal(got[2], want[2]), f"replay {replay}: cache"
        _case(gpu, 3, 16, 8, 128, [700 + replay, 33, 4096], 24 + replay)   # other work between replays
    del graph


def test_static_decode_refuses_records_beyond_the_fixed_scratch(gpu):
    """refused on the host before any launch. The caches are allocated at the
    full capacity the call names (2 x 4 GiB), so that even a regression in the
    refusal could not make the kernel read past them"""
    import torch
    B, H, KV, D = 1, 8, 8, 128
    max_pos = (1 << 21) - 1            # 1024 chunks x 8 kv heads x 4160 B > 32 MiB
    cap = max_pos + 1
    q = torch.zeros((B, H, D), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((B, KV, D), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((B, H, D), dtype=torch.float32, device="cuda")
    kc = torch.empty((B, KV, cap, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty((B, KV, cap, D), dtype=torch.bfloat16, device="cuda")
    g = torch.ones(D, dtype=torch.float32, device="cuda")
    pos = torch.tensor([max_pos], dtype=torch.int32, device="cuda")
    a = _args(gpu, q, k, k, out, kc, vc, pos, max_pos, H, KV, D, g, g, g)
    say("aigpu_decode_attention_static refusal", dict(max_pos=max_pos))
    assert gpu.lib().aigpu_decode_attention_static(C.byref(a)) == 0
    assert "fixed scratch" in gpu.last_error()
