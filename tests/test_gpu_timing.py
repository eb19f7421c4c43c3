"""The timing entry points bench.py reports from: they run the decode step's
own kernels, so their outputs are checked like any other entry point.

- bench_decode: the prompt's last step gives the first token; after the
  warm-up the position is rewound to the first decode position, so the K
  timed steps give greedy tokens 2 .. K+1 of generate() on the same prompt.
- time_projection / time_attention: positive device times, the algorithmic
  byte counts of the stated formulas, and argument errors.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6, n_heads=6,
            n_kv_heads=2, max_seq_len=256, rope_theta=10000.0, tie_word_embeddings=False)


@pytest.fixture(scope="module")
def tiny(hip):
    m = hip.LlamaModel.new_random(hip.LlamaConfig(**TINY), 3)
    yield m
    m.free()


def test_bench_decode_tokens_are_greedy(hip, orc, tiny):
    print("[case] bench_decode vs generate_greedy, tiny GQA model", flush=True)
    prompt = orc.prompt_ids(2, 40, TINY["vocab_size"])
    want = tiny.generate_greedy(prompt, 25)
    ms, toks = tiny.bench_decode(prompt, 5, 24)
    assert ms > 0
    assert np.array_equal(toks, want[1:25])


def test_time_projection_bytes(hip, tiny):
    import esolearn_amd.llama as EL
    h, ffn, V = TINY["hidden_size"], TINY["intermediate_size"], TINY["vocab_size"]
    hd = h // TINY["n_heads"]
    qd, kvd = TINY["n_heads"] * hd, TINY["n_kv_heads"] * hd
    kp = lambda k: (k + 15) // 16 * 16  # int8 row stride
    want = {EL.T_QKV: (qd + 2 * kvd) * kp(h) + 4 + 4 * h + 4 * (qd + 2 * kvd),
            EL.T_O: h * kp(qd) + 4 + 4 * qd + 4 * h,
            EL.T_GATE: 2 * ffn * kp(h) + 8 + 4 * h + 4 * ffn,
            EL.T_DOWN: h * kp(ffn) + 4 + 4 * ffn + 4 * h,
            EL.T_LM_HEAD: V * kp(h) + 4 + 4 * h + 4 * V}
    for tid, b in want.items():
        us, got = tiny.time_projection(tid, 8)
        assert us > 0 and got == b, (tid, got, b)


def test_time_attention_bytes_and_errors(hip, tiny):
    hd = TINY["hidden_size"] // TINY["n_heads"]
    kvd, qd = TINY["n_kv_heads"] * hd, TINY["n_heads"] * hd
    for ctx in (1, 17, 200):
        us, b = tiny.time_attention(ctx, 8)
        assert us > 0 and b == 8 * ctx * kvd + 8 * qd
    with pytest.raises(hip.ScryHipError):
        tiny.time_attention(TINY["max_seq_len"] + 1, 4)
    with pytest.raises(hip.ScryHipError):
        tiny.time_attention(0, 4)


@pytest.mark.parametrize("quant", ["per_tensor", "block32"])
def test_bench_qgemv_dist_gemm_path(hip, quant):
    """The micro-benchmark's GEMM path (2) and the automatic route above 16
    rows form the GEMM input as matmul_i8_f32 does (digit planes for per-tensor
    scales, bf16 planes for block-32) and return positive times and the
    algorithmic weight bytes."""
    import esolearn_amd.llama as EL
    q = EL.QUANT_PER_TENSOR if quant == "per_tensor" else EL.QUANT_BLOCK32
    print(f"[case] bench_qgemv_dist gemm path, {quant}", flush=True)
    for path in (2, 0):
        per, us, b = EL.bench_qgemv_dist(40, 1024, 768, q, path, n_bufs=2, warmup=2, iters=8, group=4)
        print(f"[time] path {path}: {us:.2f} us, {b:.0f} B", flush=True)
        assert us > 0 and (per > 0).all()
        assert b >= 1024 * 768
