"""best_times.md and LINK.md from session.json.

Same output formats as the reference's renderers (reference
scripts/render_best_times.py:12-60 and scripts/render_link_md.py:13-66): one
row per kernel of the common, standard and full sets, one column per chip
bucket, `ms (speedup×)` cells and `—` where a chip has no correct run; LINK.md
lists each chip's kernels with a link to the source that implements them.
The kernel list comes from the registries (mlx/kernels/<set>/registry.py)
instead of the reference's metal/kernels/ tree, and the links point at the HIP
source files in this repository, relative to its root.  Chip columns are
every bucket present in session.json (e.g. `amd-instinct-mi355x`) plus the
reference's Apple buckets, so a session.json carried over from the reference
renders unchanged."""
from __future__ import annotations

import json
from pathlib import Path

from . import helpers as H

APPLE_CHIPS = ["apple-m1", "apple-m2", "apple-m3", "apple-m4", "apple-m5"]


def _chips(session: dict) -> list[str]:
    extra = sorted(c for c in session if c not in APPLE_CHIPS)
    return extra + APPLE_CHIPS


def _cell(session: dict, chip: str, name: str) -> str:
    entry = session.get(chip, {}).get(name)
    if not entry:
        return "—"
    ms, sp = entry.get("best_time_ms"), entry.get("speedup_vs_mlx")
    if not isinstance(ms, (int, float)) or not isinstance(sp, (int, float)) or sp <= 0:
        return "—"
    return f"{ms:.3f} ({sp:.2f}×)"


def _short(chip: str) -> str:
    """Column title: M1 .. M5 for the Apple buckets (as the reference), the
    bucket key otherwise."""
    return chip.split("-")[-1].upper() if chip in APPLE_CHIPS else chip


def render_best_times(session: dict, kernels: list[tuple[str, str]]) -> str:
    chips = _chips(session)
    lines = [
        "# MetalBench Best Times",
        "",
        "Best kernel time + speedup vs the reference implementation per chip. "
        "`—` = not yet benchmarked on that chip.",
        "Auto-generated from `session.json` by `./bench --update-md`. Do not hand-edit.",
        "",
        "| kernel | set | " + " | ".join(_short(c) for c in chips) + " |",
        "|---|---|" + "---|" * len(chips),
    ]
    for setname, name in kernels:
        cells = " | ".join(_cell(session, c, name) for c in chips)
        lines.append(f"| `{name}` | {setname} | {cells} |")
    covered = ", ".join(f"{_short(c)} ({len(session.get(c, {}))})" for c in chips
                        if session.get(c))
    lines += ["", f"_{len(kernels)} kernels total. Chips covered: {covered or 'none'}._"]
    return "\n".join(lines) + "\n"


def render_link_md(session: dict, kernels: list[tuple[str, str]], sources: dict) -> str:
    """`sources`: kernel name -> repository-relative path of its source (or None)."""
    chips = _chips(session)
    lines = [
        "# LINK.md",
        "",
        f"Per-chip kernel source links — {len(kernels)} kernels × {len(chips)} chips.",
        "Chips without benchmark data show kernels as plain text (no link).",
        "",
        "Auto-generated from `session.json` + the kernel registries by `./bench --update-md`. "
        "Do not hand-edit.",
        "",
    ]
    for chip in chips:
        has_data = bool(session.get(chip))
        lines.append(f"## {chip}" + ("" if has_data else " _(no data)_"))
        lines.append("")
        for _, name in kernels:
            path = sources.get(name) if has_data else None
            lines.append(f"- [{name}]({path})" if path else f"- `{name}`")
        lines.append("")
    return "\n".join(lines)


def kernel_sources(kernels: list[tuple[str, str]]) -> dict:
    out = {}
    for _, name in kernels:
        p = H.find_kernel_source(name)
        try:
            out[name] = str(p.relative_to(H.REPO_ROOT)) if p else None
        except ValueError:
            out[name] = None
    return out


def update_markdown(session_path=None, out_dir=None) -> bool:
    """Write best_times.md and LINK.md next to session.json (or into out_dir)."""
    sp = Path(session_path) if session_path else H.SESSION_PATH
    if not sp.exists():
        return False
    session = json.loads(sp.read_text())
    kernels = H.all_kernels()
    out = Path(out_dir) if out_dir else H.REPO_ROOT
    (out / "best_times.md").write_text(render_best_times(session, kernels))
    (out / "LINK.md").write_text(render_link_md(session, kernels, kernel_sources(kernels)))
    return True
