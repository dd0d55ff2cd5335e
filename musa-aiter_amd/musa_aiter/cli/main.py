"""``list-ops`` and ``trace`` subcommands (reference musa_aiter/cli/main.py:74-83, :197-221).

``list-ops [--family F] [--json]`` prints the capability registry, where every
KV row names the ``rocm-hip`` backend.  ``trace -- CMD ...`` runs CMD as a
child process with ``MUSA_AITER_TRACE_DISPATCH=1`` so each hot-path call
prints its dispatch record.
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys

from musa_aiter import registry


def _list_ops(args: argparse.Namespace) -> int:
    caps = registry.list_capabilities(family=args.family)
    if args.json:
        print(json.dumps({c.name: registry.as_dict()[c.name] for c in caps}, indent=2))
        return 0
    width = max((len(c.name) for c in caps), default=4)
    for cap in caps:
        print(f"{cap.name:<{width}}  {cap.family:<8} {cap.status:<11} backends={','.join(cap.backends)} "
              f"dtypes={','.join(cap.dtypes)}")
    return 0


def _trace(args: argparse.Namespace) -> int:
    cmd = list(args.command)
    if cmd and cmd[0] == "--":
        cmd = cmd[1:]
    if not cmd:
        print("trace: missing command", file=sys.stderr)
        return 2
    env = dict(os.environ, MUSA_AITER_TRACE_DISPATCH="1")
    return subprocess.call(cmd, env=env)


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(prog="musa-aiter", description="MI355X KV-cache movement backend")
    sub = parser.add_subparsers(dest="cmd", required=True)
    p_list = sub.add_parser("list-ops", help="print registered operator capabilities")
    p_list.add_argument("--family", default=None)
    p_list.add_argument("--json", action="store_true")
    p_list.set_defaults(func=_list_ops)
    p_trace = sub.add_parser("trace", help="run a command with dispatch tracing enabled")
    p_trace.add_argument("command", nargs=argparse.REMAINDER)
    p_trace.set_defaults(func=_trace)
    args = parser.parse_args(argv)
    return int(args.func(args))


if __name__ == "__main__":
    raise SystemExit(main())
