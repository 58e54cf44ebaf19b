"""Writes the golden vectors under tests/golden/ from the reference's own code, compiled in this container.

oracle/Makefile's `ref` target builds oracle/_ref/libfnkv_ref.so from the reference checkout's sources where they lie
(ggml/src/ggml-quants.c, ggml/src/ggml-impl.h, fn/quant/kv_q8_ref.cpp) and oracle/ref_exports_*.{c,cpp}; this script
calls it and saves inputs with the reference's outputs as .npz fixtures (data only). Run it where /root/reference
exists: `python tests/golden/make_golden.py`. The GPU box never runs it; the tests read the committed fixtures.

Fixtures:
  q8_0_golden.npz   quantize_row_q8_0_ref (ggml-quants.c:274-297) on
                      stress: kv_q8_stress_rows(0x6b5638, 8) (kv_q8_ref.cpp:99-169; the seed of qa2_test.cpp:1011)
                      allf16: every finite fp16 value, in bit order, as fp32 (1,984 blocks: each exponent range)
                      ties:   blocks whose x * id land exactly on k + 0.5 (roundf's ties away from zero)
                      rows:   seeded fp16 K/V rows, N(0, 1) with 4 of 256 channels x8 (BASELINE's distribution)
                      nonfinite: fp16 rows holding NaN and +-inf among finite values (first, middle, last and
                              whole-block NaNs, inf alone, both together, seeded placements)
                    each as x (fp32), qs (int8 codes) and d (fp16 bits), plus the dequantized values
                    (dequantize_row_q8_0, ggml-quants.c:551-565)
  f16_golden.npz    ggml_compute_fp32_to_fp16 (ggml-impl.h:414-438) on 40,000 seeded fp32 bit patterns plus edge
                    values; ggml_compute_fp16_to_fp32 (ggml-impl.h:391-412) on all 65,536 halves
  kv8_golden.npz    FNFL's own KV8 rule kv_q8_quantize (kv_q8_ref.cpp:72-93) on the stress, fp16 and non-finite rows
  act_golden.npz    FNFL's int8 activation format act_quantize_ref (fn/quant/act_ref.cpp:8-29) on seeded rows of the
                    DA-TC output width (3,072), exact ties (x id = k + 0.5), zero, subnormal, huge, NaN and inf runs
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def ref_q8_0(x):
    R = O.ref()
    x = np.ascontiguousarray(x, np.float32)
    blk = np.empty((x.size // 32, 34), np.uint8)
    R.fnkv_ref_q8_0_quantize(O._ptr(x), O._ptr(blk), x.size)
    qs, d = O.from_block_q8_0(blk)
    y = np.empty(x.size, np.float32)
    R.fnkv_ref_q8_0_dequantize(O._ptr(blk), O._ptr(y), x.size)
    return qs, d, y


def stress_rows():
    R = O.ref()
    n = R.fnkv_ref_stress_rows(0x6B5638, 8, None, 0)
    s = np.empty(n, np.float32)
    R.fnkv_ref_stress_rows(0x6B5638, 8, O._ptr(s), n)
    return s


def baseline_rows(seed, n_rows, d=256):
    """fp16 rows ~ N(0, 1) with 4 of the 256 channels scaled x8 (fixed by seed)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n_rows, d)).astype(np.float32)
    ch = rng.choice(d, 4, replace=False)
    x[:, ch] *= 8.0
    return x.astype(np.float16).astype(np.float32)


def nonfinite_rows():
    """fp16 rows (whole 256-value rows, 8 blocks) holding NaN and +-inf beside finite values: a NaN first, in the
    middle (after a larger value), last and everywhere in its block, an inf alone, NaN and inf together, and seeded
    random placements. ggml's MAX macro (a > b ? a : b) lets a NaN restart the block's running max, and leaves it NaN
    only from the block's last place; a NaN or inf times id rounds to NaN, whose int8 store keeps the low byte of
    x86's 0x80000000: code 0."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((24, 256)).astype(np.float32)
    x[:, rng.choice(256, 4, replace=False)] *= 8.0
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    x[0, 0] = nan                       # first in block 0
    x[0, 32 + 31] = nan                 # last in block 1: the block's amax NaN
    x[1, 5], x[1, 3] = nan, 40.0        # a larger value before the NaN: dropped from the max
    x[1, 64 + 17], x[1, 64 + 30] = nan, nan
    x[2, 0:32] = nan                    # a whole block
    x[2, 32 + 7] = inf                  # inf alone: d inf, id 0
    x[2, 64 + 9] = -inf
    x[3, 3], x[3, 20] = inf, nan        # inf before the NaN: the max restarts after it
    x[3, 32 + 3], x[3, 32 + 20] = nan, -inf
    x[4, 31], x[4, 30] = 0.0, nan       # the NaN's followers all zero
    x[4, 32:64] = 0.0
    x[4, 32 + 31] = nan
    for r in range(5, 24):
        m = rng.random(256)
        x[r, m < 0.03] = nan
        x[r, (m >= 0.03) & (m < 0.05)] = inf
        x[r, (m >= 0.05) & (m < 0.06)] = -inf
    return x.astype(np.float16).astype(np.float32).reshape(-1)


def tie_blocks():
    out = []
    # amax 127 -> d = 1, id = 1: x = k + 0.5 exactly
    for sgn in (1.0, -1.0):
        v = np.array([127.0] + [sgn * (k + 0.5) for k in range(0, 124, 4)], np.float32)[:32]
        out.append(v)
    # amax 63.5 -> d = 0.5, id = 2: x = (k + 0.5) / 2
    v = np.array([63.5] + [((k % 127) + 0.5) / 2.0 * (1 if k % 2 else -1) for k in range(31)], np.float32)
    out.append(v)
    # amax 12.7 -> d = 0.1 (inexact), id = 1 / d: near-ties
    v = np.array([12.7] + [(k + 0.5) * 0.1 for k in range(31)], np.float32)
    out.append(v)
    return np.concatenate(out).astype(np.float32)


def act_inputs():
    """Runs of 32 for the activation format: seeded rows, ties, and edge runs."""
    rng = np.random.default_rng(20261202)
    runs = [rng.uniform(-3.0, 3.0, size=4 * 3072).astype(np.float32)]
    runs.append(rng.standard_normal(3072).astype(np.float32) * np.float32(1e-3))
    # amax 127: id = 1, x = k + 0.5 exactly (ties to even); amax 63.5: id = 2
    runs.append(np.array([127.0] + [(k % 127) + 0.5 for k in range(31)], np.float32))
    runs.append(np.array([-63.5] + [-((k % 63) + 0.5) / 2.0 for k in range(31)], np.float32))
    runs.append(np.zeros(32, np.float32))
    runs.append(np.full(32, 1e-42, np.float32) * np.arange(1, 33, dtype=np.float32))
    runs.append(np.linspace(-3e38, 3e38, 32, dtype=np.float32))
    nan = rng.uniform(-1.0, 1.0, 32).astype(np.float32)
    nan[[3, 17]] = np.nan
    runs.append(nan)
    runs.append(np.full(32, np.nan, np.float32))
    inf = rng.uniform(-1.0, 1.0, 32).astype(np.float32)
    inf[5] = np.inf
    runs.append(inf)
    return np.concatenate(runs).astype(np.float32)


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libfnkv_ref.so missing: run `make -C oracle ref` first")
    R = O.ref()
    fix = {}
    h = np.arange(65536, dtype=np.uint16)
    finite = h[(h & 0x7C00) != 0x7C00]
    sets = {
        "stress": stress_rows(),
        "allf16": O.f16_to_f32(finite)[: (finite.size // 32) * 32],
        "ties": tie_blocks(),
        "rows": baseline_rows(20261201, 64).reshape(-1),
        "nonfinite": nonfinite_rows(),
    }
    for name, x in sets.items():
        qs, d, y = ref_q8_0(x)
        fix[f"{name}_x"] = x
        fix[f"{name}_qs"] = qs
        fix[f"{name}_d"] = d
        fix[f"{name}_y"] = y
    np.savez_compressed(os.path.join(HERE, "q8_0_golden.npz"), **fix)

    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=40_000, dtype=np.uint64).astype(np.uint32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001,
                     3 * 2.0**-25, 2.0**-14, 2.0**-14 * (1 - 2.0**-11), np.inf, -np.inf, 1.0 + 2.0**-11,
                     1.0 + 3 * 2.0**-11, 1e-40], np.float32)
    xf = np.concatenate([bits.view(np.float32), edge]).astype(np.float32)
    hf = np.empty(xf.size, np.uint16)
    R.fnkv_ref_f32_to_f16(O._ptr(xf), xf.size, O._ptr(hf))
    wf = np.empty(65536, np.float32)
    R.fnkv_ref_f16_to_f32(O._ptr(h), h.size, O._ptr(wf))
    np.savez_compressed(os.path.join(HERE, "f16_golden.npz"), f32=xf, f16=hf, halves_f32_bits=wf.view(np.uint32))

    kv = {}
    for name in ("stress", "rows", "nonfinite"):
        x = np.ascontiguousarray(sets[name], np.float32)
        codes = np.empty(x.size, np.int8)
        sc = np.empty(x.size // 64, np.uint16)
        R.fnkv_ref_kv8_quantize(O._ptr(x), x.size, O._ptr(codes), O._ptr(sc))
        kv[f"{name}_x"] = x
        kv[f"{name}_codes"] = codes
        kv[f"{name}_scales"] = sc
    np.savez_compressed(os.path.join(HERE, "kv8_golden.npz"), **kv)
    act = act_inputs()
    codes = np.empty(act.size, np.int8)
    sc = np.empty(act.size // 16, np.float32)
    R.fnkv_ref_act_quantize(O._ptr(act), 1, act.size, O._ptr(codes), O._ptr(sc))
    np.savez_compressed(os.path.join(HERE, "act_golden.npz"), x=act, codes=codes, scales_bits=sc.view(np.uint32))
    for f in ("q8_0_golden.npz", "f16_golden.npz", "kv8_golden.npz", "act_golden.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
