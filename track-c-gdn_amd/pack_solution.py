"""Pack a definition's solution into one ``solution.json`` and unpack it again.

Counterpart of the reference's ``scripts/pack_solution.py:34-84`` (one copy
per definition directory).  That script reads ``config.toml`` ([solution]
name / definition / author, [build] language / entry_point /
destination_passing_style, config.toml:1-9), builds a ``BuildSpec`` and calls
``flashinfer_bench.agents.pack_solution_from_files`` on the solution's source
directory, then writes the ``Solution`` as indented JSON.  ``flashinfer_bench``
is an external, unpinned dependency that is not part of the reference tree, so
this module writes the document itself with the fields the reference passes at
its call site (pack_solution.py:52-72):

    {"name", "definition", "author", "description",
     "spec": {"language", "target_hardware", "entry_point",
              "destination_passing_style"},
     "sources": [{"path", "content"}, ...]}

Differences, each forced by what the solution is here:

* ``sources`` holds every text file the entry point needs: the definition's
  ``kernel.py`` and ``config.toml``, the package's Python modules, the HIP
  sources under ``csrc/`` and ``include/gdn_hip.h``, at their paths relative
  to the repository root.  The reference packs one directory holding a single
  self-contained ``kernel.py``.
* ``spec.entry_point`` is rewritten to that root-relative path
  (``track-c-gdn_amd/<definition>/kernel.py::run``), so it resolves inside
  the unpacked tree.
* ``spec.target_hardware`` is ``["gfx950"]``; the reference hard-codes
  ``["cuda"]`` (pack_solution.py:53).
* ``spec.language`` is ``python``: a Python entry file over a HIP library.
  The reference accepts ``triton`` or ``cuda`` and raises ``ValueError``
  otherwise (pack_solution.py:44-49); here ``python`` is the one accepted
  value, under the same error.

The library is not packed (it is machine code).  After unpacking, build it
with ``python <root>/track-c-gdn_amd/build.py`` (hipcc, gfx950).

Usage: ``python track-c-gdn_amd/pack_solution.py <definition> [-o out.json]``
and ``python track-c-gdn_amd/pack_solution.py --unpack solution.json DEST``.
"""

from __future__ import annotations

import argparse
import json
import re
import sys
from pathlib import Path
from typing import Dict, List, Optional

try:
    import tomllib
except ImportError:       # Python < 3.11
    import tomli as tomllib

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
DEFINITIONS = ("gdn_decode_qk4_v8_d128_k_last", "gdn_prefill_qk4_v8_d128_k_last")
LANGUAGES = ("python",)
TARGET_HARDWARE = ["gfx950"]
PACKAGE_FILES = ("__init__.py", "_capi.py", "decode.py", "prefill.py", "inputs.py", "build.py")


def load_config(definition_dir: Path) -> dict:
    """``config.toml`` of a definition directory (pack_solution.py:24-31)."""
    path = Path(definition_dir) / "config.toml"
    if not path.exists():
        raise FileNotFoundError(f"Config file not found: {path}")
    with open(path, "rb") as f:
        return tomllib.load(f)


def _local_includes(path: Path) -> List[str]:
    return re.findall(r'^\s*#\s*include\s+"([^"]+)"', path.read_text(), flags=re.M)


def solution_files(definition_dir: Path) -> List[Path]:
    """Every file the definition's entry point needs, in a fixed order."""
    definition_dir = Path(definition_dir).resolve()
    files = [definition_dir / "config.toml", definition_dir / "kernel.py"]
    files += [PKG_DIR / name for name in PACKAGE_FILES]
    csrc = PKG_DIR / "csrc"
    files += sorted(csrc.glob("*.hip")) + sorted(csrc.glob("*.h"))
    files += sorted((ROOT / "include").glob("*.h"))
    for f in files:
        if not f.is_file():
            raise FileNotFoundError(f"Source file not found: {f}")
    return files


def pack_solution(definition_dir: Path, output_path: Optional[Path] = None,
                  description: str = "") -> Path:
    """Write ``solution.json`` for one definition directory; returns its path."""
    definition_dir = Path(definition_dir).resolve()
    config = load_config(definition_dir)
    sol, build = config["solution"], config["build"]
    language = build["language"]
    if language not in LANGUAGES:
        raise ValueError(f"Unsupported language: {language}")
    entry_file, _, entry_fn = build["entry_point"].partition("::")
    rel_dir = definition_dir.relative_to(ROOT).as_posix()
    sources: List[Dict[str, str]] = [
        {"path": f.relative_to(ROOT).as_posix(), "content": f.read_text()}
        for f in solution_files(definition_dir)]
    doc = {
        "name": sol["name"],
        "definition": sol["definition"],
        "author": sol["author"],
        "description": description,
        "spec": {
            "language": language,
            "target_hardware": list(TARGET_HARDWARE),
            "entry_point": f"{rel_dir}/{entry_file}::{entry_fn}",
            "destination_passing_style": bool(build.get("destination_passing_style", True)),
        },
        "sources": sources,
    }
    if output_path is None:
        output_path = definition_dir / "solution.json"
    output_path = Path(output_path)
    output_path.write_text(json.dumps(doc, indent=2))
    return output_path


def unpack_solution(solution_path: Path, dest: Path) -> Path:
    """Write the sources of a packed solution under ``dest``; returns the
    entry file's path.  Paths must be relative and stay inside ``dest``."""
    doc = json.loads(Path(solution_path).read_text())
    dest = Path(dest).resolve()
    for src in doc["sources"]:
        rel = Path(src["path"])
        target = (dest / rel).resolve()
        if rel.is_absolute() or dest not in target.parents:
            raise ValueError(f"Source path escapes the destination: {src['path']}")
        target.parent.mkdir(parents=True, exist_ok=True)
        target.write_text(src["content"])
    entry_file = doc["spec"]["entry_point"].partition("::")[0]
    return dest / entry_file


def main(argv: Optional[List[str]] = None) -> int:
    parser = argparse.ArgumentParser(description="Pack a solution into solution.json")
    parser.add_argument("definition", nargs="?", choices=DEFINITIONS)
    parser.add_argument("-o", "--output", type=Path, default=None,
                        help="output path (default: <definition dir>/solution.json)")
    parser.add_argument("--unpack", nargs=2, metavar=("SOLUTION_JSON", "DEST"), type=Path)
    args = parser.parse_args(argv)
    try:
        if args.unpack:
            entry = unpack_solution(*args.unpack)
            print(f"Solution unpacked: entry file {entry}")
            return 0
        if args.definition is None:
            parser.error("a definition or --unpack is required")
        out = pack_solution(PKG_DIR / args.definition, args.output)
        doc = json.loads(out.read_text())
        print(f"Solution packed: {out}")
        print(f"  Name: {doc['name']}")
        print(f"  Definition: {doc['definition']}")
        print(f"  Author: {doc['author']}")
        print(f"  Language: {doc['spec']['language']}")
        print(f"  Sources: {len(doc['sources'])}")
        return 0
    except Exception as e:       # same reporting as the reference's main()
        print(f"Error: {e}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    sys.exit(main())
