"""Developer toolkit for the library's ops: list, info, doctor, verify,
benchmark, compare, visualize, profile (the command set of the reference's
`custom_cuda_cli`, custom_cuda/cli/app.py:101-512). Run it as
`python -m custom_cuda_kernals_amd.cli`. Typer and rich load only when the
CLI runs, not when the package is imported."""

from __future__ import annotations

__all__ = ["main"]


def main() -> None:
    from custom_cuda_kernals_amd.cli.app import app

    app()
