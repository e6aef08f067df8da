"""The solution packer (counterpart of the reference's scripts/pack_solution.py:34-84).

CPU: fields follow config.toml, every source is packed byte for byte and is
self-contained (each local #include resolves inside the pack), unpacking
restores the tree, the reference's error cases raise the same exception types.
GPU: the unpacked entry files, run in a fresh process against the library
built from the same sources, match the oracle on the operator bars.
"""

import json
import os
import shutil
import subprocess
import sys
import textwrap

import pytest

from conftest import ROOT, pkg_module

DEFS = ("gdn_decode_qk4_v8_d128_k_last", "gdn_prefill_qk4_v8_d128_k_last")
PKG = ROOT / "track-c-gdn_amd"


def _packer():
    return pkg_module("pack_solution")


@pytest.mark.parametrize("definition", DEFS)
def test_pack_fields_follow_config(tmp_path, definition):
    ps = _packer()
    out = ps.pack_solution(PKG / definition, tmp_path / "solution.json")
    doc = json.loads(out.read_text())
    cfg = ps.load_config(PKG / definition)
    assert doc["name"] == cfg["solution"]["name"]
    assert doc["definition"] == cfg["solution"]["definition"] == definition
    assert doc["author"] == cfg["solution"]["author"]
    spec = doc["spec"]
    assert spec["language"] == cfg["build"]["language"] == "python"
    assert spec["target_hardware"] == ["gfx950"]
    assert spec["destination_passing_style"] is False
    assert spec["entry_point"] == f"track-c-gdn_amd/{definition}/kernel.py::run"
    paths = [s["path"] for s in doc["sources"]]
    assert len(paths) == len(set(paths))
    for p in (f"track-c-gdn_amd/{definition}/kernel.py", "include/gdn_hip.h",
              "track-c-gdn_amd/csrc/gdn_prefill.hip", "track-c-gdn_amd/build.py"):
        assert p in paths
    for s in doc["sources"]:
        assert (ROOT / s["path"]).read_text() == s["content"]
    assert not any(p.endswith(".so") for p in paths)


def test_packed_sources_are_self_contained(tmp_path):
    ps = _packer()
    doc = json.loads(ps.pack_solution(PKG / DEFS[1], tmp_path / "s.json").read_text())
    paths = {s["path"] for s in doc["sources"]}
    for s in doc["sources"]:
        if s["path"].endswith((".hip", ".h")):
            for inc in ps._local_includes(ROOT / s["path"]):
                here = os.path.normpath(os.path.join(os.path.dirname(s["path"]), inc))
                assert here in paths or f"include/{inc}" in paths, (s["path"], inc)


def test_unpack_restores_the_tree(tmp_path):
    ps = _packer()
    sol = ps.pack_solution(PKG / DEFS[0], tmp_path / "s.json")
    entry = ps.unpack_solution(sol, tmp_path / "out")
    assert entry == (tmp_path / "out" / f"track-c-gdn_amd/{DEFS[0]}/kernel.py").resolve()
    for s in json.loads(sol.read_text())["sources"]:
        assert (tmp_path / "out" / s["path"]).read_text() == (ROOT / s["path"]).read_text()


def test_unpack_rejects_escaping_paths(tmp_path):
    ps = _packer()
    for bad in ("../evil.py", "/tmp/evil.py"):
        sol = tmp_path / "bad.json"
        sol.write_text(json.dumps({"spec": {"entry_point": "x.py::run"},
                                   "sources": [{"path": bad, "content": "x"}]}))
        with pytest.raises(ValueError):
            ps.unpack_solution(sol, tmp_path / "out")


def test_reference_error_cases(tmp_path):
    ps = _packer()
    with pytest.raises(FileNotFoundError):          # pack_solution.py:27-28
        ps.pack_solution(tmp_path, tmp_path / "s.json")
    d = tmp_path / "def"
    d.mkdir()
    (d / "config.toml").write_text(
        '[solution]\nname = "x"\ndefinition = "y"\nauthor = "z"\n'
        '[build]\nlanguage = "triton"\nentry_point = "kernel.py::run"\n')
    with pytest.raises(ValueError):                 # pack_solution.py:48-49
        ps.pack_solution(d, tmp_path / "s.json")


def test_cli_pack_and_unpack(tmp_path):
    out = tmp_path / "sol.json"
    r = subprocess.run([sys.executable, str(PKG / "pack_solution.py"), DEFS[1], "-o", str(out)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "Solution packed" in r.stdout
    r = subprocess.run([sys.executable, str(PKG / "pack_solution.py"), "--unpack", str(out),
                        str(tmp_path / "tree")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert (tmp_path / "tree" / f"track-c-gdn_amd/{DEFS[1]}/kernel.py").exists()


_RUN_UNPACKED = textwrap.dedent("""
    import sys, torch
    from importlib.machinery import SourceFileLoader
    tree, repo = sys.argv[1], sys.argv[2]
    sys.path.insert(0, repo)
    from oracle import gdn_oracle as O
    dec = SourceFileLoader("u_dec", tree + "/track-c-gdn_amd/gdn_decode_qk4_v8_d128_k_last/kernel.py").load_module()
    pre = SourceFileLoader("u_pre", tree + "/track-c-gdn_amd/gdn_prefill_qk4_v8_d128_k_last/kernel.py").load_module()
    pkg = sys.modules["track_c_gdn_amd"]
    assert pkg.__file__.startswith(tree), pkg.__file__
    import importlib
    inp = importlib.import_module("track_c_gdn_amd.inputs")
    dev = torch.device("cuda:0")
    to = lambda x: {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}
    def check(o, s, o_ref, s_ref):
        torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
        s = s.cpu().double()
        rel = float((s - s_ref).norm() / s_ref.norm())
        assert rel <= 1e-3, rel
    x = inp.decode_inputs(8, seed=77); g = to(x)
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")
    print("unpacked decode B=8", flush=True)
    o, s = dec.run(*[g[n] for n in names], g["scale"]); torch.cuda.synchronize()
    check(o, s, *O.decode_step(*[x[n] for n in names], x["scale"]))
    x = inp.prefill_inputs([100, 37], seed=78, with_state=True); g = to(x)
    names = names + ("cu_seqlens",)
    print("unpacked prefill lens=[100, 37]", flush=True)
    o, s = pre.run(*[g[n] for n in names], g["scale"]); torch.cuda.synchronize()
    check(o, s, *O.prefill_recurrent(*[x[n] for n in names], x["scale"]))
    print("unpacked solution ok", flush=True)
""")


@pytest.mark.gpu
def test_unpacked_solution_runs(tmp_path, device):
    ps = _packer()
    tree = tmp_path / "tree"
    for d in DEFS:
        ps.unpack_solution(ps.pack_solution(PKG / d, tmp_path / f"{d}.json"), tree)
    # the library built from these same sources (checked byte for byte above)
    shutil.copy2(PKG / "libgdn_hip.so", tree / "track-c-gdn_amd" / "libgdn_hip.so")
    script = tmp_path / "run_unpacked.py"
    script.write_text(_RUN_UNPACKED)
    r = subprocess.run([sys.executable, "-u", str(script), str(tree.resolve()), str(ROOT)],
                       capture_output=True, text=True, timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert "unpacked solution ok" in r.stdout
