"""frisk-opt for this build: parse textual tile IR, run the frisk passes,
print the result.

The reference's tools/frisk-opt/frisk-opt.cpp is MlirOptMain over its pass
registry (include/Dialect/Frisk/Transforms/Passes.td).  This driver runs the
same passes of this package, with their names and options:

  --frisk-normalize-layout-ir[='target=gfx950']
  --frisk-infer-layouts[='analysis-only dump-analysis exact-combination-limit=N
                          beam-width=N max-expanded-states=N cost-profile=FILE|NAME
                          target=gfx950']
  --frisk-export-execution[='output=FILE minify']

Passes run in command-line order on the module read from the input file (or
stdin, `-`).  The module is printed to stdout (or -o FILE) afterwards, as
mlir-opt does; --frisk-export-execution without output= writes the packet to
stdout instead of the module.  dump-analysis writes the constraint listing to
stderr.  cost-profile= takes a profile file or the name of one shipped in
frisk_amd/cost_profiles (e.g. cdna4-calibrated-v1, fitted to kernel times by
frisk_amd/calibrate.py).  -verify-each verifies the module after every pass.  Errors go to
stderr as `<file>:<line>:<col>: error: ...` (parse) or `error: ...` (passes)
and the exit status is 1.

Usage: python -m frisk_amd.opt [input] [passes...] [-o FILE] [-verify-each]
                               [--mlir-print-debuginfo]
"""
from __future__ import annotations

import json
import re
import shlex
import sys

from . import _ir, create_context

PASSES = ("frisk-normalize-layout-ir", "frisk-infer-layouts", "frisk-export-execution")


class OptError(Exception):
    pass


def _options(text: str) -> dict:
    """`'a b=1 c=x'` -> {"a": True, "b": "1", "c": "x"} (MLIR pass options)."""
    out = {}
    for tok in shlex.split(text or ""):
        key, eq, val = tok.partition("=")
        out[key] = val if eq else True
    return out


def _int(opts, key, default):
    v = opts.get(key, default)
    try:
        return int(v)
    except (TypeError, ValueError):
        raise OptError(f"option {key} needs an integer (got {v!r})")


def run_pass(name: str, opts: dict, module, streams) -> bool:
    """Run one pass; returns False when the module must not be printed."""
    fr = _ir().frisk
    known = {
        "frisk-normalize-layout-ir": {"target"},
        "frisk-infer-layouts": {"analysis-only", "dump-analysis", "exact-combination-limit",
                                "beam-width", "max-expanded-states", "cost-profile", "target"},
        "frisk-export-execution": {"output", "minify"},
    }[name]
    unknown = set(opts) - known
    if unknown:
        raise OptError(f"--{name}: unknown option(s) {', '.join(sorted(unknown))}")
    try:
        if name == "frisk-normalize-layout-ir":
            fr.normalize_layout_ir(module, opts.get("target"))
            return True
        if name == "frisk-infer-layouts":
            profile = None
            if opts.get("cost-profile"):
                from .calibrate import load_profile
                profile = load_profile(opts["cost-profile"])
            report = fr.infer_layouts(
                module, opts.get("target"),
                exact_combination_limit=_int(opts, "exact-combination-limit", 256),
                beam_width=_int(opts, "beam-width", 32),
                max_expanded_states=_int(opts, "max-expanded-states", 65536),
                analysis_only=bool(opts.get("analysis-only")), cost_profile=profile)
            if opts.get("dump-analysis"):
                err = streams["err"]
                err.write("frisk-infer-layouts analysis\n")
                for line in report["graph"]:
                    err.write(line + "\n")
                err.write(f"solution: {report['status']} method={report['method']} "
                          f"cost={report['cost']} variables={report['variables']} "
                          f"combinations={report['combinations']} expanded={report['expanded']}\n")
                for a in report["assignments"]:
                    err.write(f"assignment {a}\n")
                for c in report["conversions"]:
                    err.write(f"conversion {c}\n")
            if report["status"] == "failed":
                raise OptError(f"frisk-infer-layouts: {report.get('failure', 'failed')}")
            return True
        packet = fr.export_execution(module)
        if opts.get("minify"):
            packet = json.dumps(json.loads(packet), separators=(",", ":"))
        if opts.get("output"):
            with open(opts["output"], "w") as f:
                f.write(packet + "\n")
            return True
        streams["out"].write(packet + "\n")
        return False
    except ValueError as e:
        raise OptError(f"--{name}: {e}") from None


def parse_args(argv):
    args = {"input": "-", "output": None, "passes": [], "verify_each": False, "debuginfo": False}
    it = iter(argv)
    for a in it:
        if a in ("-o", "--o"):
            args["output"] = next(it, None)
            if args["output"] is None:
                raise OptError("-o needs a file name")
        elif a in ("-verify-each", "--verify-each"):
            args["verify_each"] = True
        elif a in ("--mlir-print-debuginfo", "-mlir-print-debuginfo"):
            args["debuginfo"] = True
        elif a.startswith("-") and a != "-":
            name, eq, val = a.lstrip("-").partition("=")
            if name not in PASSES:
                raise OptError(f"unknown option or pass '{a}' (passes: {', '.join(PASSES)})")
            args["passes"].append((name, _options(val)))
        else:
            args["input"] = a
    return args


def main(argv=None, stdout=None, stderr=None) -> int:
    stdout = stdout or sys.stdout
    stderr = stderr or sys.stderr
    try:
        args = parse_args(list(sys.argv[1:] if argv is None else argv))
        src = sys.stdin.read() if args["input"] == "-" else open(args["input"]).read()
    except (OptError, OSError) as e:
        stderr.write(f"frisk-opt: error: {e}\n")
        return 1
    ir = _ir()
    ctx = create_context()
    where = "<stdin>" if args["input"] == "-" else args["input"]
    try:
        module = ir.frisk.parse_module(src, ctx)
    except ValueError as e:
        m = re.match(r"(\d+):(\d+): (.*)", str(e), re.S)
        stderr.write(f"{where}:{m[1]}:{m[2]}: error: {m[3]}\n" if m else f"{where}: error: {e}\n")
        return 1
    module.context = ctx
    if not module.verify():
        stderr.write(f"{where}: error: {module.verify_diagnostic()}\n")
        return 1
    show = True
    try:
        for name, opts in args["passes"]:
            show = run_pass(name, opts, module, {"out": stdout, "err": stderr}) and show
            if args["verify_each"] and not module.verify():
                raise OptError(f"--{name}: the module does not verify afterwards: "
                               f"{module.verify_diagnostic()}")
    except OptError as e:
        stderr.write(f"error: {e}\n")
        return 1
    if show:
        text = ir.frisk.print_module(module, debug_info=args["debuginfo"]) + "\n"
        if args["output"]:
            with open(args["output"], "w") as f:
                f.write(text)
        else:
            stdout.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
