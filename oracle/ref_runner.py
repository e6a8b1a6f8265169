"""Run the reference's own CPU operators in a child process (test infrastructure).

``make -C oracle ref`` compiles the reference's extension source
(cpp/src/bindings.cpp) without CUDA into oracle/_ref/cudaforge_ref.so; its CPU
operator implementations (bindings.cpp:238-329) are the reference semantics
as shipped. That library registers the same ``cudaforge`` operator namespace
as this build's extension, so it can never share a process with
cuda_force_amd: this module is executed as a script in a fresh interpreter.

Two modes:

  python -m oracle.ref_runner run REQUEST.npz RESULT.npz
      REQUEST holds ``op`` (str) and input arrays ``in0, in1, ...`` plus an
      optional float ``scalar``; bf16 inputs are stored as uint16 bits with
      ``dtype`` = "bf16". RESULT holds ``out0, out1, ...`` (bf16 results as
      uint16 bits).

  python -m oracle.ref_runner time OP --shape ... --dtype ... --seconds S
      Times the reference operator on seeded synthetic inputs and prints one
      JSON line (the "reference" CPU baseline in bench.py).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REF_LIBRARY = Path(__file__).resolve().parent / "_ref" / "cudaforge_ref.so"


def available() -> bool:
    return REF_LIBRARY.exists()


def _load_reference():
    import torch

    if "cuda_force_amd" in sys.modules:
        raise RuntimeError("the reference library cannot share a process with cuda_force_amd")
    torch.ops.load_library(str(REF_LIBRARY))
    return torch


def _to_tensor(torch, array, dtype: str):
    import numpy as np

    if dtype == "bf16" and array.dtype == np.uint16:
        return torch.from_numpy(array.astype(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(array)


def _from_tensor(tensor):
    import numpy as np
    import torch

    tensor = tensor.detach().contiguous().cpu()
    if tensor.dtype == torch.bfloat16:
        return tensor.view(torch.int16).numpy().astype(np.uint16)
    return tensor.numpy()


def run_request(request_path: str, result_path: str) -> None:
    import numpy as np

    torch = _load_reference()
    with np.load(request_path, allow_pickle=False) as req:
        op = str(req["op"])
        dtype = str(req["dtype"]) if "dtype" in req.files else "f32"
        inputs = []
        i = 0
        while f"in{i}" in req.files:
            inputs.append(_to_tensor(torch, req[f"in{i}"], dtype))
            i += 1
        scalar = float(req["scalar"]) if "scalar" in req.files else None
    fn = getattr(torch.ops.cudaforge, op)
    result = fn(*inputs, scalar) if scalar is not None else fn(*inputs)
    outputs = list(result) if isinstance(result, (list, tuple)) else [result]
    np.savez(result_path, **{f"out{k}": _from_tensor(t) for k, t in enumerate(outputs)})


def call_reference(op: str, inputs: list, dtype: str = "f32", scalar: float | None = None,
                   workdir: str | None = None) -> list:
    """Run one reference operator in a child process and return its outputs."""
    import subprocess
    import tempfile

    import numpy as np

    with tempfile.TemporaryDirectory(dir=workdir) as tmp:
        req = os.path.join(tmp, "req.npz")
        res = os.path.join(tmp, "res.npz")
        payload = {"op": np.array(op), "dtype": np.array(dtype)}
        for k, arr in enumerate(inputs):
            payload[f"in{k}"] = np.ascontiguousarray(arr)
        if scalar is not None:
            payload["scalar"] = np.array(scalar, dtype=np.float64)
        np.savez(req, **payload)
        root = str(Path(__file__).resolve().parent.parent)
        subprocess.run(
            [sys.executable, "-m", "oracle.ref_runner", "run", req, res],
            check=True,
            cwd=root,
            env={**os.environ, "PYTHONPATH": root},
        )
        with np.load(res, allow_pickle=False) as out:
            return [out[f"out{k}"] for k in range(len(out.files))]


def time_reference(op: str, shape: list[int], dtype: str, seconds: float, threads: int) -> dict:
    """Median wall time of the reference CPU operator on seeded inputs."""
    torch = _load_reference()
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    tdtype = {"f32": torch.float32, "bf16": torch.bfloat16}[dtype]
    if op == "quantize_int8":
        x = torch.randn(*shape, generator=gen).to(tdtype)
        fn = lambda: torch.ops.cudaforge.quantize_int8(x)  # noqa: E731
    elif op == "dequantize_int8":
        x = torch.randn(*shape, generator=gen)
        q, s = torch.ops.cudaforge.quantize_int8(x)
        fn = lambda: torch.ops.cudaforge.dequantize_int8(q, s)  # noqa: E731
    elif op == "rmsnorm":
        x = torch.randn(*shape, generator=gen).to(tdtype)
        w = (1 + 0.02 * torch.randn(shape[-1], generator=gen)).to(tdtype)
        fn = lambda: torch.ops.cudaforge.rmsnorm(x, w, 1e-6)  # noqa: E731
    elif op == "softmax":
        # Config 2's logits: N(0, 4) with the causal -inf mask of row index
        # mod cols, as the GPU step times them.
        rows, cols = shape[0], shape[-1]
        x = 2.0 * torch.randn(rows, cols, generator=gen)
        masked = torch.arange(cols)[None, :] > (torch.arange(rows) % cols)[:, None]
        x = x.masked_fill(masked, float("-inf")).to(tdtype)
        fn = lambda: torch.ops.cudaforge.softmax(x)  # noqa: E731
    elif op == "lora_linear":
        m, k, n, r = shape
        x = torch.randn(m, k, generator=gen).to(tdtype)
        w = (0.02 * torch.randn(k, n, generator=gen)).to(tdtype)
        a = (torch.randn(k, r, generator=gen) / 64).to(tdtype)
        b = (0.02 * torch.randn(r, n, generator=gen)).to(tdtype)
        fn = lambda: torch.ops.cudaforge.lora_linear(x, w, a, b, 2.0)  # noqa: E731
    else:
        raise ValueError(f"unknown op {op}")
    for _ in range(2):
        fn()
    samples = []
    started = time.perf_counter()
    while len(samples) < 5 or time.perf_counter() - started < seconds:
        t0 = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t0)
    return {
        "op": op,
        "shape": shape,
        "dtype": dtype,
        "median_s": statistics.median(samples),
        "runs": len(samples),
        "threads": torch.get_num_threads(),
        "cpu_count": os.cpu_count(),
    }


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    sub = parser.add_subparsers(dest="mode", required=True)
    run = sub.add_parser("run")
    run.add_argument("request")
    run.add_argument("result")
    timing = sub.add_parser("time")
    timing.add_argument("op")
    timing.add_argument("--shape", type=int, nargs="+", required=True)
    timing.add_argument("--dtype", default="f32")
    timing.add_argument("--seconds", type=float, default=10.0)
    timing.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    args = parser.parse_args(argv)
    if args.mode == "run":
        run_request(args.request, args.result)
    else:
        print(json.dumps(time_reference(args.op, args.shape, args.dtype, args.seconds, args.threads)))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
