"""GPU parity of the prefill attentionMixer in one call (aigpu_prefill_mixer):
the q, k, v projections (the k and v GEMMs carrying QK-RMSNorm -> RoPE -> KV
append as their epilogue), flash attention over the bf16 cache, the output
gate and the o projection, against the oracle's composition of its pinned
pieces: matmul_nt (apply, LocalModel.hpp:1052-1078), qk_norm_rope (:2608-2648),
attention_strided over the cached history and the new fp32 rows
(Kernels.hpp:130-168), output_gate (:2660-2665) and matmul_nt again (:2667).

Bar: the bf16 attention bar (max-abs <= 2e-3, rel-L2 <= 1e-3) on the mixer's
output, whose scale is kept near 1 (weights ~ N(0, 1/fan_in)); the new cache
rows within bf16 rounding (2^-8 of the largest) of the oracle's normed,
rotated keys and of the projected values."""
import numpy as np
import pytest

from common import assert_bf16_parity, bf16_normal, gammas
from gpu_util import dev_bf16, dev_f32, host, say
from oracle import oracle as O
from test_gpu_matmul import quantise, to_device

pytestmark = pytest.mark.gpu


def weight(n, k, kind, seed, tag):
    """(stored form, scales, dense fp32 it stands for) of an [n][k] weight ~ N(0, 1/k)"""
    src = (O.fill_normal((n, k), seed, tag) / np.sqrt(k)).astype(np.float32)
    if kind == "f32":
        return src, None, src
    if kind == "bf16":
        bits = O.pack_bf16(src).reshape(n, k)
        return bits, None, O.unpack_bf16(bits).reshape(n, k)
    codes, scales = quantise(src, kind)
    return codes, scales, O.dequant(codes, scales, kind)


def run(gpu, kind="bf16", count=70, start=25, hidden=256, H=8, KV=2, D=128, gate=False, norm=True,
        rope=True, rot=None, biases=False, window=0, seed=3, accumulate=False, x_scale=1.0):
    import torch
    qs = 2 * D if gate else D
    cap = start + count + 5
    rot = rot or D
    x = O.fill_normal((count, hidden), seed, "x") * np.float32(x_scale)
    shapes = {"q": (H * qs, hidden), "k": (KV * D, hidden), "v": (KV * D, hidden), "o": (hidden, H * D)}
    dev, ref = {}, {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        stored, scales, _ = weight(n, k, kind, seed + 10 * i, "w" + name)
        bias = O.fill_normal((n,), seed + 10 * i, "b" + name) * 0.1 if biases else None
        dev[name] = {"w": to_device(stored), "kind": kind, "out": n, "in": k,
                     "scales": None if scales is None else dev_f32(scales),
                     "bias": None if bias is None else dev_f32(bias)}
        ref[name] = (stored, scales, bias)
    gq = gammas(D, seed, "q_norm") if norm else None
    gk = gammas(D, seed, "k_norm") if norm else None
    fr = O.rotary_frequencies(rot, 1e6) if rope else None
    hkb, hk = bf16_normal((KV, start, D), seed, "k_cache")
    hvb, hv = bf16_normal((KV, start, D), seed, "v_cache")
    kc = np.zeros((KV, cap, D), np.uint16)
    vc = np.zeros((KV, cap, D), np.uint16)
    kc[:, :start] = hkb
    vc[:, :start] = hvb

    # attentionMixer through the oracle function whose composition the
    # reference's FP64 model pins (tests/test_oracle_fixture_model.py), over
    # the widened bf16 history in the reference's position-major fp32 cache
    layer = {name: (stored, kind, scales, bias) for name, (stored, scales, bias) in ref.items()}
    layer.update(q_norm=gq, k_norm=gk, window=window)
    keys = np.zeros((start + count, KV * D), np.float32)
    vals = np.zeros((start + count, KV * D), np.float32)
    keys[:start] = hk.transpose(1, 0, 2).reshape(start, KV * D)
    vals[:start] = hv.transpose(1, 0, 2).reshape(start, KV * D)
    mcfg = dict(heads=H, kv_heads=KV, head_dim=D, rotary_dims=rot, eps=1e-6, freqs=fr)
    want, _, kn = O.attention_mixer(x, layer, keys, vals, start, mcfg, q_stride=qs, gate=gate)
    v = vals[start:start + count].reshape(count, KV, D)
    base = O.fill_normal((count, hidden), seed, "residual") if accumulate else None
    if accumulate:
        want = want + base

    key_cache, value_cache = dev_bf16(kc), dev_bf16(vc)
    out = dev_f32(base) if accumulate else torch.zeros((count, hidden), dtype=torch.float32, device="cuda")
    say("prefill mixer", dict(kind=kind, count=count, start=start, hidden=hidden, H=H, KV=KV, D=D, gate=gate,
                              norm=norm, rope=rope, rot=rot, biases=biases, window=window, accumulate=accumulate))
    gpu.prefill_mixer(dev_f32(x), dev, out, key_cache, value_cache, start, H, KV, D,
                      q_norm=None if gq is None else dev_f32(gq), k_norm=None if gk is None else dev_f32(gk),
                      freqs=None if fr is None else dev_f32(fr), rotary_dims=rot, window=window,
                      output_gate=gate, accumulate=accumulate, check=True)
    got = host(out)
    assert_bf16_parity(want, got, f"mixer {kind}")
    gk_all, gv_all = host(key_cache), host(value_cache)
    new_k = gk_all[:, start:start + count].transpose(1, 0, 2)
    new_v = gv_all[:, start:start + count].transpose(1, 0, 2)
    assert np.abs(new_k - kn).max() <= np.abs(kn).max() * 2 ** -8, "appended keys"
    assert np.abs(new_v - v).max() <= np.abs(v).max() * 2 ** -8, "appended values"
    assert (host(key_cache)[:, :start] == O.unpack_bf16(hkb).reshape(KV, start, D)).all(), "history kept"
    assert not gk_all[:, start + count:].any(), "rows past the prefill untouched"


@pytest.mark.parametrize("kind", ["f32", "bf16", "q8", "q4"])
def test_weight_encodings(gpu, kind):
    run(gpu, kind)


@pytest.mark.parametrize("count,start", [(1, 0), (16, 0), (130, 0), (300, 97)])
def test_counts_and_history(gpu, count, start):
    run(gpu, "bf16", count=count, start=start)


@pytest.mark.parametrize("H,KV,D,rot,biases,hidden,gate,acc", [
    (16, 8, 128, None, False, 64, False, False), (8, 8, 128, None, True, 64, False, False),
    (32, 16, 64, 32, True, 64, False, False), (2, 1, 64, None, False, 2048, False, True),
    (2, 1, 64, 32, True, 2048, True, False)])
def test_fused_kv_projection(gpu, H, KV, D, rot, biases, hidden, gate, acc):
    """8192 rows and 2 KV D = 2048 k and v columns make 256 tiles of 256 x 256:
    k and v run as one DMA GEMM over both weights, then kv_epilogue_kernel. At
    H D = 2048 the q projection takes the DMA GEMM too and its bf16 split of x
    is reused; at H D = 1024 the pair splits x itself. At hidden = 2048 the o
    projection has 256 such tiles too (here with 2 heads of 64, to keep the
    oracle's projections short; k and v then take two launch_gemm_kv calls): the flash kernel then writes its bf16
    operand images in place of fp32 rows (with the output gate applied first
    when there is one), and the residual add rides on the GEMM. A window of 64
    keeps the oracle's attention short."""
    run(gpu, "bf16", count=8192, start=40, hidden=hidden, H=H, KV=KV, D=D, rot=rot, biases=biases, window=64,
        gate=gate, accumulate=acc)


def test_head_dim_64_partial_rotary_and_biases(gpu):
    run(gpu, "bf16", D=64, H=4, KV=2, rot=32, biases=True)


def test_output_gate_window_and_residual_add(gpu):
    run(gpu, "bf16", gate=True, window=33, accumulate=True)


def test_no_qk_norm_no_rope(gpu):
    run(gpu, "bf16", norm=False, rope=False)


def test_rejects_mismatched_shapes(gpu):
    import torch
    x = torch.zeros((4, 256), dtype=torch.float32, device="cuda")
    w = {n: {"w": torch.zeros(256 * 256 * 2, dtype=torch.uint8, device="cuda"), "kind": "bf16", "out": 256}
         for n in "qkvo"}
    kc = torch.zeros((2, 8, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((4, 256), dtype=torch.float32, device="cuda")
    gpu.prefill_mixer(x, w, out, kc, kc, 0, 2, 2, 128)   # 2 heads of 128: every shape fits
    with pytest.raises(RuntimeError, match="weight shapes"):   # 4 heads: q needs 512 rows
        gpu.prefill_mixer(x, w, out, kc, kc, 0, 4, 2, 128)
