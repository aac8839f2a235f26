"""Writes tests/golden/randint_vectors.json: tl.randint(seed, offsets) values.

The reference's stochastic rounding draws its random bits with Triton's
``tl.randint`` (shared_ffi/sr_triton.py:11).  Triton is a third-party
dependency (the reference pins torch 2.4.0, i.e. Triton 3.0.x; this container
has Triton 3.6.0, whose triton/language/random.py has the same Philox4x32-10
randint/randint4x definition).  This script runs the installed Triton's own
``tl.randint`` in interpreter mode on the CPU -- no reference code is imported
-- and stores the outputs as golden vectors for the CPU oracle and the HIP
kernels.

Run:  python tests/golden/make_randint_vectors.py
"""
import json
import os

os.environ["TRITON_INTERPRET"] = "1"

import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402


@triton.jit
def _randint_kernel(out_ptr, offs_ptr, seed, N: tl.constexpr):
    i = tl.arange(0, N)
    offs = tl.load(offs_ptr + i)
    tl.store(out_ptr + i, tl.randint(seed, offs))


def main():
    cases = []
    seeds = [0, 42, 123, 124, 2**31 + 7, 2**32 + 5, 0xDEADBEEFCAFE]
    offset_sets = {
        "0..63": list(range(64)),
        "near_2^31": [2**31 - 3 + i for i in range(8)] + [2**32 - 2, 2**32 - 1],
        "int64": [2**32, 2**32 + 1, 5 * 2**32 + 77, 2**40 + 123456],
        "sparse": [1000, 16777343, 16777344, 393215, 99991, 3 * 10**8 + 17, 7, 65536],
    }
    for seed in seeds:
        for name, offs in offset_sets.items():
            n = 1
            while n < len(offs):
                n *= 2
            o = torch.tensor(offs + [0] * (n - len(offs)), dtype=torch.int64)
            if name != "int64" and max(offs) < 2**31:
                o = o.to(torch.int32)
            out = torch.empty(n, dtype=torch.int32)
            _randint_kernel[(1,)](out, o, seed, N=n)
            vals = [v & 0xFFFFFFFF for v in out.tolist()[: len(offs)]]
            cases.append({"seed": seed, "offsets": offs, "set": name,
                          "offset_dtype": str(o.dtype).replace("torch.", ""),
                          "randint": vals})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "randint_vectors.json")
    with open(path, "w") as f:
        json.dump({"generator": f"triton {triton.__version__} tl.randint, TRITON_INTERPRET=1",
                   "cases": cases}, f, indent=1)
    print("wrote", path, len(cases), "cases")


if __name__ == "__main__":
    main()
