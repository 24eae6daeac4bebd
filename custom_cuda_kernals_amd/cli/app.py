"""The CLI's commands: thin orchestration over `registry` (what an op is)
and `runners` (how to test, time and profile it); rendering is here.
Command set of the reference's toolkit (custom_cuda/cli/app.py:101-512)."""

from __future__ import annotations

import difflib
import time
from pathlib import Path

import typer
from rich import box
from rich.console import Console
from rich.panel import Panel
from rich.table import Table
from rich.text import Text

from custom_cuda_kernals_amd import __version__
from custom_cuda_kernals_amd.cli.registry import REGISTRY, OpSpec, get_op, list_ops
from custom_cuda_kernals_amd.cli.runners import RESULTS, load_bench, run_bench, run_profile, run_pytest, time_pair

console = Console()
err = Console(stderr=True)
OK, FAIL, WARN = "[bold green]OK[/bold green]", "[bold red]FAIL[/bold red]", "[bold yellow]WARN[/bold yellow]"
PEAK_GBPS = 8000.0

app = typer.Typer(name="custom_cuda_kernals_amd", no_args_is_help=False, add_completion=False,
                  help="Developer toolkit for the MI355X (gfx950) activation-path kernels.")

COMMANDS = [
    ("list", "List the ops with their id and title."),
    ("doctor", "Inspect the environment (ROCm, hipcc, PyTorch HIP, GPU arch, OCP FP8, native library)."),
    ("info OP", "Show an op's specification, files, tests and C entry points."),
    ("verify [OP]", "Run the op's tests (GPU tests when a GPU is visible, CPU tests otherwise)."),
    ("benchmark OP", "Run bench.py for the op and show time, bandwidth and fraction of 8 TB/s."),
    ("compare OP", "Time the kernel against the reference's eager formula on the GPU."),
    ("visualize OP", "Chart the op's measured bandwidth against the 8 TB/s peak (PNG)."),
    ("profile OP", "Capture a rocprofv3 kernel trace of the op and show the top kernels."),
    ("help", "Show this command list."),
]


def _resolve(op_id: str) -> OpSpec:
    spec = get_op(op_id)
    if spec is not None:
        return spec
    near = difflib.get_close_matches(op_id, REGISTRY.keys(), n=3)
    hint = f" Did you mean: {', '.join(near)}?" if near else " Run `list` to see the op ids."
    err.print(f"[bold red]Error:[/bold red] unknown op {op_id!r}.{hint}")
    raise typer.Exit(code=1)


def _require_gpu() -> None:
    import torch

    if not torch.cuda.is_available():
        err.print("[bold red]Error:[/bold red] no HIP device visible. Run `doctor` to diagnose.")
        raise typer.Exit(code=1)


def _help_table() -> None:
    console.print(Panel(f"[bold cyan]custom_cuda_kernals_amd[/bold cyan] v{__version__} — hand-written HIP "
                        "kernels for MI355X behind the reference's C ABI", box=box.ROUNDED, border_style="cyan"))
    t = Table(box=box.SIMPLE_HEAVY, header_style="bold cyan")
    t.add_column("Command", style="bold")
    t.add_column("Description")
    for c, d in COMMANDS:
        t.add_row(c, d)
    console.print(t)
    console.print("[dim]Op ids: " + ", ".join(s.id for s in list_ops()) + "[/dim]")


@app.callback(invoke_without_command=True)
def _root(ctx: typer.Context, version: bool = typer.Option(False, "--version", help="Show the version.")) -> None:
    if version:
        console.print(f"custom_cuda_kernals_amd {__version__}")
        raise typer.Exit()
    if ctx.invoked_subcommand is None:
        _help_table()
        raise typer.Exit()


@app.command(name="help")
def help_cmd() -> None:
    """Show all commands."""
    _help_table()


@app.command(name="list")
def list_cmd() -> None:
    """List the ops with their id and title."""
    t = Table(title="Ops", box=box.SIMPLE_HEAVY, header_style="bold cyan")
    t.add_column("#", justify="right")
    t.add_column("id", style="bold cyan")
    t.add_column("Title")
    t.add_column("Python API")
    for s in list_ops():
        t.add_row(str(s.number), s.id, s.title, ", ".join(s.python_api))
    console.print(t)


@app.command()
def doctor() -> None:
    """Inspect the environment the kernels need."""
    from custom_cuda_kernals_amd.cli.env_checks import run_checks

    checks = run_checks()
    t = Table(title="Environment", box=box.SIMPLE_HEAVY, header_style="bold cyan")
    t.add_column("Check")
    t.add_column("Status", justify="center")
    t.add_column("Detail")
    badge = {"ok": OK, "fail": FAIL, "warn": WARN}
    for c in checks:
        t.add_row(c.name, badge[c.status], c.detail)
    console.print(t)
    n_fail = sum(c.status == "fail" for c in checks)
    if n_fail:
        console.print(f"\n[bold red]{n_fail} check(s) failed.[/bold red]")
        raise typer.Exit(code=1)
    console.print("\n[bold green]Everything the kernels need is in place.[/bold green]")


@app.command()
def info(op: str = typer.Argument(..., help="Op id (see `list`).")) -> None:
    """Show an op's specification."""
    s = _resolve(op)
    body = Text()
    for head, val in (("Purpose", s.purpose), ("Formula", s.formula), ("Memory profile", s.memory_profile),
                      ("Dtypes", ", ".join(s.dtypes)), ("Target", s.target)):
        body.append(head + "\n", style="bold underline")
        body.append(val + "\n\n")
    body.append("Design\n", style="bold underline")
    for d in s.design:
        body.append(f"  • {d}\n")
    body.append("\nFiles\n", style="bold underline")
    body.append(f"  python API:   custom_cuda_kernals_amd.kernels.{', '.join(s.python_api)}\n")
    body.append(f"  C ABI:        {', '.join(s.c_entry_points)} (include/custom_kernels_amd.h)\n")
    body.append(f"  sources:      {', '.join(s.sources)}\n")
    body.append(f"  tests:        {', '.join(s.test_files)}\n")
    body.append(f"  bench.py ops: {', '.join(s.bench_ops)}\n")
    body.append(f"  reference:    {', '.join(s.reference)}\n")
    console.print(Panel(body, title=f"[bold cyan]{s.number:02d}[/bold cyan] — {s.title}", border_style="cyan"))


@app.command()
def verify(op: str | None = typer.Argument(None, help="Op id; omit to run every test."),
           cpu: bool = typer.Option(False, "--cpu", help="Run the CPU tests even when a GPU is visible."),
           timeout: int = typer.Option(1200, "--timeout", help="Max seconds for pytest.")) -> None:
    """Run the op's tests."""
    import torch

    files, title = (["tests/"], "every op") if op is None else (list(_resolve(op).test_files), op)
    marker = "gpu" if torch.cuda.is_available() and not cpu else "not gpu"
    with console.status(f"[cyan]pytest -m '{marker}' for {title}...[/cyan]"):
        r = run_pytest(files, marker, timeout)
    t = Table(box=box.SIMPLE_HEAVY, header_style="bold cyan")
    t.add_column("Metric")
    t.add_column("Value", justify="right")
    for k, v in (("Passed", r.passed), ("Failed", r.failed), ("Errors", r.errors), ("Skipped / deselected", r.skipped),
                 ("Duration", f"{r.duration_s:.2f}s"), ("Marker", marker)):
        t.add_row(k, str(v))
    console.print(t)
    if not r.ok:
        for line in [ln for ln in r.stdout.splitlines() if ln.startswith(("FAILED", "ERROR"))][:25]:
            console.print(f"  [red]{line}[/red]")
        console.print(f"\n{FAIL} — tests failed for {title}.")
        raise typer.Exit(code=1)
    console.print(f"\n{OK} — all tests passed for {title}.")


def _bench_rows(line: dict) -> list[tuple[str, dict]]:
    return list(line.get("ops", {}).items())


def _bench_table(spec: OpSpec, line: dict, full: bool = False) -> None:
    if full:  # every recorded field, one table per bench.py op
        for name, r in _bench_rows(line):
            t = Table(title=name, box=box.SIMPLE_HEAVY, header_style="bold cyan")
            t.add_column("field")
            t.add_column("value", justify="right", overflow="fold")
            for k, v in r.items():
                if isinstance(v, dict):
                    for k2, v2 in v.items():
                        t.add_row(f"{k}.{k2}", str(v2))
                else:
                    t.add_row(k, str(v))
            console.print(t)
        return
    t = Table(title=f"{spec.id} (bench.py)", box=box.SIMPLE_HEAVY, header_style="bold cyan")
    for c in ("op", "workload", "µs / launch", "GB/s", "of 8 TB/s", "per call µs (flush, binding)"):
        t.add_column(c, justify="left" if c in ("op", "workload") else "right",
                     overflow="fold" if c in ("op", "workload") else "ellipsis")
    for name, r in _bench_rows(line):
        pc = (r.get("per_call") or {}).get("median_us")
        t.add_row(name, r["workload"], f"{r['us']:.2f}", f"{r['GB_per_s']:.0f}", f"{100 * r['frac_of_8TBps']:.1f} %",
                  f"{pc:.2f}" if pc is not None else "-")
    console.print(t)


@app.command()
def benchmark(op: str = typer.Argument(..., help="Op id (see `list`)."),
              rerun: bool = typer.Option(False, "--rerun", help="Run bench.py even if a result is stored."),
              full: bool = typer.Option(False, "--full", help="Show every recorded field, not just the key ones."),
              steps: int = typer.Option(100, "--steps", help="Timed launches per bench.py op."),
              timeout: int = typer.Option(900, "--timeout", help="Max seconds for bench.py.")) -> None:
    """Run bench.py for the op (graph-replayed, >= 2 GiB buffer rotation), or show its stored result."""
    spec = _resolve(op)
    line = None if rerun else load_bench(spec.id)
    if line is None:
        _require_gpu()
        with console.status(f"[cyan]bench.py --ops {','.join(spec.bench_ops)}...[/cyan]"):
            try:
                line = run_bench(spec.id, spec.bench_ops, steps, timeout)
            except Exception as e:
                err.print(f"[bold red]{e}[/bold red]")
                raise typer.Exit(code=1) from e
    else:
        console.print(f"[dim]stored result (cli_results/bench_{spec.id}.json); --rerun measures again[/dim]")
    _bench_table(spec, line, full)


@app.command()
def compare(op: str = typer.Argument(..., help="Op id (see `list`)."),
            iters: int = typer.Option(20, "--iters", help="Timed calls of each.")) -> None:
    """Time the kernel against the reference's eager formula (torch on the GPU)."""
    spec = _resolve(op)
    _require_gpu()
    target = spec.build_target("cuda")
    r = time_pair(target, iters=iters)
    t = Table(title=target.description, box=box.SIMPLE_HEAVY, header_style="bold cyan")
    for c in ("eager torch µs", "kernel µs", "speedup", "kernel GB/s", "of 8 TB/s"):
        t.add_column(c, justify="right")
    style = "bold green" if r["speedup"] >= 1.0 else "bold red"
    t.add_row(f"{r['eager_us']:.1f}", f"{r['kernel_us']:.1f}", f"[{style}]{r['speedup']:.2f}x[/{style}]",
              f"{r['kernel_GB_per_s']:.0f}", f"{100 * r['kernel_GB_per_s'] / PEAK_GBPS:.1f} %")
    console.print(t)
    console.print("[dim]One call per event pair, including the Python wrapper and binding; bench.py's graph-replayed "
                  "timing excludes them.[/dim]")


@app.command()
def visualize(op: str = typer.Argument(..., help="Op id (see `list`)."),
              rerun: bool = typer.Option(False, "--rerun", help="Run bench.py even if a result is stored."),
              output: Path | None = typer.Option(None, "--output", "-o", help="PNG path.")) -> None:  # noqa: B008
    """Chart the op's measured bandwidth against the 8 TB/s peak."""
    spec = _resolve(op)
    line = None if rerun else load_bench(spec.id)
    if line is None:
        _require_gpu()
        with console.status("[cyan]no stored result: running bench.py...[/cyan]"):
            line = run_bench(spec.id, spec.bench_ops, 100, 900)
    import matplotlib

    matplotlib.use("Agg")
    import matplotlib.pyplot as plt

    rows = _bench_rows(line)
    names = [n for n, _ in rows]
    frac = [100 * r["frac_of_8TBps"] for _, r in rows]
    fig, ax = plt.subplots(figsize=(max(5, 1.6 * len(rows) + 2), 4))
    ax.bar(names, frac, color="#2a7ab0")
    ax.axhline(100, color="black", lw=1)
    ax.axhline(75, color="#c0392b", lw=1, ls="--", label="75 % target")
    for i, (_, r) in enumerate(rows):
        ax.text(i, frac[i] + 1.5, f"{r['GB_per_s'] / 1000:.2f} TB/s\n{r['us']:.1f} µs", ha="center", fontsize=8)
    ax.set_ylabel("% of 8 TB/s HBM peak")
    ax.set_ylim(0, 110)
    ax.set_title(f"{spec.id}: achieved HBM bandwidth on one MI355X")
    ax.legend(loc="lower right")
    plt.xticks(rotation=15, ha="right", fontsize=8)
    fig.tight_layout()
    out = output or (RESULTS / f"{spec.id}_bandwidth.png")
    out.parent.mkdir(parents=True, exist_ok=True)
    fig.savefig(out, dpi=120)
    console.print(f"{OK} wrote {out}")


@app.command()
def profile(op: str = typer.Argument(..., help="Op id (see `list`)."),
            warmup: int = typer.Option(5, "--warmup", help="Calls before the profiled ones."),
            iters: int = typer.Option(10, "--iters", help="Profiled calls."),
            output: Path | None = typer.Option(None, "--output", "-o", help="Output directory."),  # noqa: B008
            timeout: int = typer.Option(600, "--timeout", help="Max seconds for rocprofv3.")) -> None:
    """Capture a rocprofv3 kernel trace of the op and show the top kernels."""
    spec = _resolve(op)
    _require_gpu()
    out = output or (RESULTS / f"profile_{spec.id}_{time.strftime('%Y%m%d_%H%M%S')}")
    with console.status(f"[cyan]rocprofv3 --kernel-trace --stats over {warmup} + {iters} calls...[/cyan]"):
        try:
            r = run_profile(spec.id, iters, out, timeout, warmup=warmup)
        except Exception as e:
            err.print(f"[bold red]{e}[/bold red]")
            raise typer.Exit(code=1) from e
    t = Table(title="Kernels by total time", box=box.SIMPLE_HEAVY, header_style="bold cyan")
    cols = [c for c in ("Name", "Calls", "AverageNs", "TotalDurationNs", "Percentage") if r.top and c in r.top[0]]
    for c in cols:
        t.add_column(c, justify="left" if c == "Name" else "right")
    for row in r.top:
        t.add_row(*[(row[c][:90] if c == "Name" else row[c]) for c in cols])
    console.print(t)
    console.print(f"{OK} trace and statistics in {r.out_dir}")
    if r.trace is not None:
        console.print(f"[dim]Timeline: {r.trace} (open in https://ui.perfetto.dev).[/dim]")
