"""``python -m aklr_amd.schema fill DEFINITION.json... --to DIR [--author NAME]`` writes each definition,
filled with this library's kernel, at ``DIR/<op>/impls/hip/<name>/<uuid>.json``; copy the files to the
same relative paths under ``aklr/ops`` (or the plugin's ``models`` directory) of an AKLR checkout.
``python -m aklr_amd.schema check FILE.json...`` lists what AKLR would reject in written files."""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

from . import AUTHOR, PackagingError, check, fill, write


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(prog="python -m aklr_amd.schema")
    sub = parser.add_subparsers(dest="command", required=True)
    f = sub.add_parser("fill", help="fill definitions with this library's kernels")
    f.add_argument("definitions", nargs="+", type=Path)
    f.add_argument("--to", type=Path, required=True)
    f.add_argument("--author", default=AUTHOR)
    c = sub.add_parser("check", help="check written schema files")
    c.add_argument("files", nargs="+", type=Path)
    args = parser.parse_args(argv)
    failed = False
    if args.command == "fill":
        for definition in args.definitions:
            try:
                print(write(fill(json.loads(definition.read_text(encoding="utf-8")), author=args.author), args.to))
            except PackagingError as e:
                failed = True
                print(f"{definition}: {e}", file=sys.stderr)
    else:
        for path in args.files:
            for problem in check(path):
                failed = True
                print(f"{path}: {problem}", file=sys.stderr)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
