"""Writes tests/golden/v2_philox.json: values of Triton's counter-based generator
(``tl.randint4x`` and ``tl.rand``, triton/language/random.py) produced by Triton's own CPU
interpreter (TRITON_INTERPRET=1).  They pin the Philox4x32 restatement in
oracle/v2_rejection.py that the V2 verification (minivllm/worker/gpu/sample/gumbel.py:72-91)
relies on.  Nothing from the reference checkout is imported or run; Triton is the
third-party library the reference calls.

Run: python tests/golden/make_v2_philox.py
"""

import json
import os
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"

import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402


@triton.jit
def _draw(out_ptr, rand_ptr, offs_ptr, seed, N: tl.constexpr):
    i = tl.arange(0, N)
    off = tl.load(offs_ptr + i)
    a, b, c, d = tl.randint4x(seed, off)
    tl.store(out_ptr + 4 * i + 0, a)
    tl.store(out_ptr + 4 * i + 1, b)
    tl.store(out_ptr + 4 * i + 2, c)
    tl.store(out_ptr + 4 * i + 3, d)
    tl.store(rand_ptr + i, tl.rand(seed, off))


def main() -> None:
    cases = []
    offsets64 = [0, 1, 7, 4095, 151935, 2**31 - 1, 2**32 + 5, 2**40 + 123]
    offsets32 = [0, 1, 7, 99, 4095, 12345, 151935, 2**31 - 1]  # power-of-two count (tl.arange)
    for seed in (1, 12345, 2**31 - 1, 2**33 + 17, 2**62 + 99):
        for dtype, offs in ((torch.int64, offsets64), (torch.int32, offsets32)):
            o = torch.tensor(offs, dtype=dtype)
            out = torch.zeros(4 * len(offs), dtype=torch.int32)
            r = torch.zeros(len(offs), dtype=torch.float32)
            _draw[(1,)](out, r, o, seed, N=len(offs))
            cases.append({
                "seed": seed,
                "offset_dtype": "int64" if dtype == torch.int64 else "int32",
                "offsets": offs,
                "randint4x": [[int(v) & 0xFFFFFFFF for v in out[4 * j:4 * j + 4].tolist()]
                              for j in range(len(offs))],
                "rand_bits": [int(v) for v in r.view(torch.int32).tolist()],
            })
    path = Path(__file__).with_name("v2_philox.json")
    path.write_text(json.dumps({"triton": triton.__version__, "cases": cases}, indent=0) + "\n")
    print(f"wrote {path} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
