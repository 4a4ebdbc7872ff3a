"""Render the parity-margin log of a GPU test run as a markdown table.

The GPU tests record every tolerance comparison (tests/helpers.py ``record``)
and, with ``LOGO_PARITY_LOG=<file>`` set, write them as JSON lines when the
session ends.  This prints one row per comparison: the test, the tensor, the
measured max and mean error, the bounds and the fraction of each bound used.

Usage: ``python tests/parity_margins.py <log.jsonl> [command that made it]``
"""

import json
import sys


def render(path, command=None):
    with open(path) as f:
        recs = [json.loads(line) for line in f if line.strip()]
    out = ["# Parity margins of the GPU tests", ""]
    if command:
        out += [f"Command: `{command}`", ""]
    out += [f"{len(recs)} comparisons.  `max` / `mean` are the measured errors against each test's reference; "
            "`used` is the error as a fraction of its bound.  Kinds other than `abs` say how `max` is scaled.", "",
            "| test | tensor | kind | max | bound | used | mean | bound | used |",
            "|---|---|---|---|---|---|---|---|---|"]
    worst_max = worst_mean = (0.0, None)
    for r in recs:
        def frac(x, b):
            return "" if not b else f"{x / b:.1%}"
        mb, nb = r.get("max_bound"), r.get("mean_bound")
        if mb:
            worst_max = max(worst_max, (r["max"] / mb, f"{r['test']} {r['tensor']}"), key=lambda t: t[0])
        if nb:
            worst_mean = max(worst_mean, (r["mean"] / nb, f"{r['test']} {r['tensor']}"), key=lambda t: t[0])
        test = (r.get("test") or "").replace("tests/", "")
        out.append(f"| {test} | {r['tensor']} | {r.get('kind', 'abs')} | {r['max']:.3e} | {mb if mb else '-'} | "
                   f"{frac(r['max'], mb)} | {r['mean']:.3e} | {nb if nb else '-'} | {frac(r['mean'], nb)} |")
    out += ["", f"Largest fraction of a max bound used: {worst_max[0]:.1%} ({worst_max[1]}).",
            f"Largest fraction of a mean bound used: {worst_mean[0]:.1%} ({worst_mean[1]})."]
    return "\n".join(out) + "\n"


if __name__ == "__main__":
    sys.stdout.write(render(sys.argv[1], " ".join(sys.argv[2:]) or None))
