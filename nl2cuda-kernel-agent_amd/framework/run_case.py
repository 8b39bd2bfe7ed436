"""Case runner CLI: verify, bench, and the verify-gated bench with a one-line
verdict.

The reference drives a case through two scripts and a runner:
skill/scripts/verify_case.py (parity of a candidate against the case's
reference, exit 0 / 1), skill/scripts/bench_case.py (timing against
torch.compile of the reference, with ``--emit-verdict`` printing one
machine-readable line and ``--strict`` turning the verdict into the exit
code), and run_on_a100.sh, which benches only after verify passes
(run_on_a100.sh:222-224).  This module keeps those commands, their
arguments and outputs, for the MI355X build:

  python nl2cuda-kernel-agent_amd/framework/run_case.py verify --case rbf
  python nl2cuda-kernel-agent_amd/framework/run_case.py bench  --case rbf --emit-verdict
  python nl2cuda-kernel-agent_amd/framework/run_case.py run    --case rbf

``--impl module:fn`` selects another candidate (default
``cases.<case>.op:candidate``); ``--baseline eager`` times the reference
without torch.compile.  ``run`` prints ``VERDICT=VERIFY_FAIL`` and exits 1
when parity fails, else the bench verdict line (exit 0, or 1 on a failed
verdict with ``--strict``).  Without a GPU every command exits 2 with a
message: there is no CPU path.
"""

import argparse
import importlib
import os
import sys

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if PKG not in sys.path:
    sys.path.insert(0, PKG)


def load_case(name):
    return importlib.import_module(f"cases.{name}").CASE


def load_impl(spec):
    mod_path, fn_name = spec.split(":")
    return getattr(importlib.import_module(mod_path), fn_name)


def _verify(case, impl):
    from framework.verify import verify_all
    ok, report = verify_all(case, impl, device="cuda")
    print(report, flush=True)
    return ok


def _bench(case, impl, baseline, emit_verdict):
    from framework.bench import compare, parse_verdict
    report, passed = compare(case, impl, device="cuda", baseline=baseline)
    print(report, flush=True)
    verdict = parse_verdict(report, passed)
    if emit_verdict:
        print(verdict, flush=True)
    return passed, verdict


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("command", choices=["verify", "bench", "run"])
    ap.add_argument("--case", required=True, help="case name, e.g. rbf")
    ap.add_argument("--impl", default=None,
                    help="candidate as module:fn (default cases.<case>.op:candidate)")
    ap.add_argument("--baseline", default="compile", choices=["compile", "eager"],
                    help="time the reference under torch.compile (default) or eagerly")
    ap.add_argument("--emit-verdict", action="store_true",
                    help="bench: print the one-line VERDICT=... summary after the report")
    ap.add_argument("--strict", action="store_true",
                    help="bench / run: exit 1 unless the verdict is PASS")
    args = ap.parse_args(argv)

    import torch
    if not torch.cuda.is_available():
        print("run_case: needs an MI355X GPU (torch.cuda.is_available() is False); "
              "there is no CPU path", file=sys.stderr)
        return 2

    case = load_case(args.case)
    impl_spec = args.impl or f"cases.{args.case}.op:candidate"
    impl = load_impl(impl_spec)
    print(f"case={args.case}  impl={impl_spec}", flush=True)

    if args.command == "verify":
        return 0 if _verify(case, impl) else 1
    if args.command == "run" and not _verify(case, impl):
        print("VERDICT=VERIFY_FAIL", flush=True)
        return 1
    passed, _ = _bench(case, impl, args.baseline,
                       emit_verdict=args.emit_verdict or args.command == "run")
    return 1 if (args.strict and not passed) else 0


if __name__ == "__main__":
    sys.exit(main())
