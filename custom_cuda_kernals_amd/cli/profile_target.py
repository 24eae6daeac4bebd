"""The program `profile` runs under rocprofv3: `warmup` calls (default 2),
then `iters` calls of one op's representative kernel call, then exit."""

from __future__ import annotations

import sys


def main(argv: list[str]) -> int:
    import torch

    from custom_cuda_kernals_amd.cli.registry import get_op

    spec = get_op(argv[0])
    if spec is None:
        print(f"unknown op {argv[0]!r}", file=sys.stderr)
        return 2
    iters = int(argv[1]) if len(argv) > 1 else 10
    warmup = int(argv[2]) if len(argv) > 2 else 2
    target = spec.build_target("cuda")
    for _ in range(warmup):
        target.kernel()
    torch.cuda.synchronize()
    for _ in range(iters):
        target.kernel()
    torch.cuda.synchronize()
    print(f"profiled {iters} calls of {target.description}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
