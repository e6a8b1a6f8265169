"""Write the golden vectors under tests/golden/ from the reference's own operators.

    make -C oracle ref                 # builds oracle/_ref/cudaforge_ref.so
    python tests/golden/make_golden.py

Every expected output here comes from the reference's CPU operator
implementations (cpp/src/bindings.cpp:238-329), compiled from the reference
source by oracle/Makefile and executed in a child process by
oracle/ref_runner.py. The reference's own test suites store no vectors (their
inputs are generated at run time), so these fixtures are seeded inputs chosen
to cover the cases those tests exercise plus the edge cases of the
quantiser's semantics: ties at .5, -0.0, all-zero blocks, a subnormal absmax
(where the reference's CPU and CUDA guards disagree), NaN and inf blocks,
ragged tails, outliers.

Inputs come from numpy's PCG64 with fixed seeds. bf16 tensors are stored as
uint16 bit patterns.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ref_runner  # noqa: E402
from oracle.floatops import f32_to_bf16_bits  # noqa: E402

OUT = Path(__file__).resolve().parent


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def quant_inputs() -> dict[str, np.ndarray]:
    cases: dict[str, np.ndarray] = {}
    for n in (1, 63, 64, 65, 1000, 4096):
        cases[f"randn_{n}"] = (rng(n).standard_normal(n) * 5.0).astype(np.float32)
    x = rng(7).standard_normal(8192).astype(np.float32)
    idx = rng(8).choice(x.size, size=82, replace=False)
    x[idx] *= 20.0
    cases["outliers_1pct"] = x
    # Ties: absmax 127 gives scale exactly 1, so x / s = x and k + 0.5 values
    # are exact ties (round half to even: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, ...).
    ties = np.zeros(128, np.float32)
    ties[0] = 127.0
    ties[1:64] = np.arange(1, 64, dtype=np.float32) - 0.5
    ties[64] = -127.0
    ties[65:128] = -(np.arange(1, 64, dtype=np.float32) - 0.5)
    cases["ties"] = ties
    # Near-ties one ulp either side of k + 0.5 with scale 1.
    near = np.zeros(192, np.float32)
    base = np.arange(63, dtype=np.float32) + 0.5
    near[0] = 127.0
    near[1:64] = np.nextafter(base, np.float32(0))
    near[64] = 127.0
    near[65:128] = np.nextafter(base, np.float32(200))
    near[128] = -127.0
    near[129:192] = -np.nextafter(base, np.float32(200))
    cases["near_ties"] = near
    # Non-unit scale with ties: absmax 63.5 -> s = 0.5, and x = k/2 + 0.25
    # gives x / s = k + 0.5.
    cases["half_scale_ties"] = np.concatenate(
        [np.array([63.5], np.float32), np.arange(-15.75, 15.75, 0.5, dtype=np.float32)[:63]]
    )
    signed_zero = np.zeros(64, np.float32)
    signed_zero[::2] = -0.0
    cases["signed_zeros"] = signed_zero
    zeros = np.concatenate([np.zeros(64, np.float32), rng(9).standard_normal(64).astype(np.float32)])
    cases["zero_block"] = zeros
    # absmax / 127 underflows to exactly zero in fp32: the CPU guard gives scale 1.
    tiny = np.zeros(64, np.float32)
    tiny[3] = np.float32(1e-45)
    tiny[5] = -np.float32(1e-45)
    cases["underflow_scale"] = tiny
    # absmax / 127 is a (nonzero) subnormal: scale stays subnormal.
    sub = np.full(64, np.float32(3e-39))
    sub[0] = np.float32(1.1e-38)
    sub[1::3] *= -1
    cases["subnormal_scale"] = sub
    nan_block = rng(10).standard_normal(128).astype(np.float32)
    nan_block[70] = np.nan
    cases["nan_block"] = nan_block
    inf_block = rng(11).standard_normal(128).astype(np.float32)
    inf_block[5] = np.inf
    inf_block[6] = -2.0
    cases["inf_block"] = inf_block
    with np.errstate(over="ignore"):
        big = rng(12).standard_normal(130).astype(np.float32) * np.float32(1e38)
    cases["huge_values"] = big
    return cases


def write_quant() -> None:
    payload: dict[str, np.ndarray] = {}
    for name, x in quant_inputs().items():
        q, s = ref_runner.call_reference("quantize_int8", [x])
        (deq,) = ref_runner.call_reference("dequantize_int8", [q, s])
        payload[f"{name}__x"] = x
        payload[f"{name}__q"] = q
        payload[f"{name}__s"] = s
        payload[f"{name}__deq"] = deq
    np.savez_compressed(OUT / "quant_f32.npz", **payload)

    payload = {}
    for n in (1, 64, 100, 2048):
        x = f32_to_bf16_bits(rng(100 + n).standard_normal(n).astype(np.float32) * 0.02)
        if n == 2048:
            idx = rng(101).choice(n, size=3, replace=False)
            x = x.copy()
            x[idx] = f32_to_bf16_bits(
                (rng(102).standard_normal(3) * 50 * 0.02).astype(np.float32)
            )
        q, s = ref_runner.call_reference("quantize_int8", [x], dtype="bf16")
        payload[f"bf16_{n}__x"] = x
        payload[f"bf16_{n}__q"] = q
        payload[f"bf16_{n}__s"] = s
    np.savez_compressed(OUT / "quant_bf16.npz", **payload)


def write_rmsnorm() -> None:
    payload: dict[str, np.ndarray] = {}
    for rows, cols in ((1, 1), (1, 64), (3, 17), (8, 128), (2, 4096), (33, 1023)):
        g = rng(rows * 1000 + cols)
        x = g.standard_normal((rows, cols)).astype(np.float32)
        w = g.standard_normal(cols).astype(np.float32)
        (y,) = ref_runner.call_reference("rmsnorm", [x, w], scalar=1e-6)
        key = f"f32_{rows}x{cols}"
        payload[f"{key}__x"], payload[f"{key}__w"], payload[f"{key}__y"] = x, w, y
    for rows, cols in ((4, 256), (2, 4096)):
        g = rng(rows * 7000 + cols)
        x = f32_to_bf16_bits(g.standard_normal((rows, cols)).astype(np.float32))
        w = f32_to_bf16_bits((1.0 + 0.02 * g.standard_normal(cols)).astype(np.float32))
        (y,) = ref_runner.call_reference("rmsnorm", [x, w], dtype="bf16", scalar=1e-6)
        key = f"bf16_{rows}x{cols}"
        payload[f"{key}__x"], payload[f"{key}__w"], payload[f"{key}__y"] = x, w, y
    np.savez_compressed(OUT / "rmsnorm.npz", **payload)


def causal_logits(rows: int, cols: int, seed: int) -> np.ndarray:
    x = (rng(seed).standard_normal((rows, cols)) * 2.0).astype(np.float32)
    col = np.arange(cols)[None, :]
    row = (np.arange(rows) % cols)[:, None]
    x[col > row] = -np.inf
    return x


def write_softmax() -> None:
    payload: dict[str, np.ndarray] = {}
    for rows, cols in ((1, 1), (1, 32), (4, 17), (8, 256), (3, 1025), (4, 4096)):
        x = rng(rows * 31 + cols).standard_normal((rows, cols)).astype(np.float32)
        (y,) = ref_runner.call_reference("softmax", [x])
        key = f"f32_{rows}x{cols}"
        payload[f"{key}__x"], payload[f"{key}__y"] = x, y
    extreme = np.array([[1000.0, 1000.0, 1000.0, 1000.0], [-1000.0, 0.0, 500.0, 1000.0]], np.float32)
    (y,) = ref_runner.call_reference("softmax", [extreme])
    payload["extreme__x"], payload["extreme__y"] = extreme, y
    x = f32_to_bf16_bits(causal_logits(64, 256, 5))
    (y,) = ref_runner.call_reference("softmax", [x], dtype="bf16")
    payload["bf16_causal_64x256__x"], payload["bf16_causal_64x256__y"] = x, y
    np.savez_compressed(OUT / "softmax.npz", **payload)


def write_lora() -> None:
    payload: dict[str, np.ndarray] = {}
    for batch, k, n, r in ((1, 8, 4, 2), (4, 64, 32, 8), (7, 129, 65, 3), (16, 256, 256, 16)):
        g = rng(batch * 100000 + k * 100 + n + r)
        x = g.standard_normal((batch, k)).astype(np.float32)
        w = g.standard_normal((k, n)).astype(np.float32)
        a = g.standard_normal((k, r)).astype(np.float32)
        b = g.standard_normal((r, n)).astype(np.float32)
        (y,) = ref_runner.call_reference("lora_linear", [x, w, a, b], scalar=0.25)
        key = f"f32_{batch}x{k}x{n}r{r}"
        for name, arr in (("x", x), ("w", w), ("a", a), ("b", b), ("y", y)):
            payload[f"{key}__{name}"] = arr
    g = rng(4242)
    x = f32_to_bf16_bits(g.standard_normal((64, 256)).astype(np.float32))
    w = f32_to_bf16_bits((0.02 * g.standard_normal((256, 128))).astype(np.float32))
    a = f32_to_bf16_bits((g.standard_normal((256, 16)) / 64).astype(np.float32))
    b = f32_to_bf16_bits((0.02 * g.standard_normal((16, 128))).astype(np.float32))
    (y,) = ref_runner.call_reference("lora_linear", [x, w, a, b], dtype="bf16", scalar=2.0)
    for name, arr in (("x", x), ("w", w), ("a", a), ("b", b), ("y", y)):
        payload[f"bf16_64x256x128r16__{name}"] = arr
    np.savez_compressed(OUT / "lora.npz", **payload)


def write_misc() -> None:
    payload: dict[str, np.ndarray] = {}
    for n in (1, 63, 64, 65, 1000, 4096):
        x = rng(500 + n).standard_normal(n).astype(np.float32)
        (s,) = ref_runner.call_reference("sum", [x])
        payload[f"sum_{n}__x"], payload[f"sum_{n}__y"] = x, s
    ones = np.ones(100_000, np.float32)
    (s,) = ref_runner.call_reference("sum", [ones])
    payload["sum_ones__x"], payload["sum_ones__y"] = ones, s
    x = np.linspace(-8, 8, 1024, dtype=np.float32)
    up = rng(600).standard_normal(1024).astype(np.float32)
    for op in ("silu", "gelu"):
        (y,) = ref_runner.call_reference(op, [x])
        payload[f"{op}__x"], payload[f"{op}__y"] = x, y
    (y,) = ref_runner.call_reference("swiglu", [x, up])
    payload["swiglu__x"], payload["swiglu__up"], payload["swiglu__y"] = x, up, y
    g = rng(700)
    x = g.standard_normal((8, 512)).astype(np.float32)
    res = g.standard_normal((8, 512)).astype(np.float32)
    w = g.standard_normal(512).astype(np.float32)
    y, summed = ref_runner.call_reference("fused_residual_rmsnorm", [x, res, w], scalar=1e-6)
    payload["frn__x"], payload["frn__res"], payload["frn__w"] = x, res, w
    payload["frn__y"], payload["frn__sum"] = y, summed
    np.savez_compressed(OUT / "misc.npz", **payload)


def main() -> int:
    if not ref_runner.available():
        print("oracle/_ref is not built; run `make -C oracle ref` first", file=sys.stderr)
        return 1
    write_quant()
    write_rmsnorm()
    write_softmax()
    write_lora()
    write_misc()
    for path in sorted(OUT.glob("*.npz")):
        print(f"{path.name}: {path.stat().st_size} bytes")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
