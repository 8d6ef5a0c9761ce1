"""AKLR schema packaging (aklr_amd.schema), on the CPU.

Pins:
- text and uuid: ``json_file_text`` and ``schema_uuid`` reproduce the text and the file name of every
  schema file the reference commits (both rules derive from the reference's code, which is not run).
- call keys: each packaged op's arguments equal those of the reference's own kernels for the contract
  (their ``run`` signatures or ``m.def`` strings), and its writes equal the schema's outputs. For
  gemm_a4w4_mxfp4, which has no committed kernel, they equal the api's parameters: the contract hides
  none of them (aklr/core/contract/op.py:548-558).
- audit: the reference's committed HIP kernels pass it. Each rule catches a violation planted in a
  copy of a packaged kernel, and accepts the lookalikes that are allowed.
- fill: every definition the reference holds for these contracts and layouts fills; the filled file
  differs from the definition only in ``kernel`` and the dropped measurements, as AKLR's export check
  requires; it passes ``check``.
Tests that read the reference skip where it is absent.
"""
from __future__ import annotations

import ast
import copy
import json
import re
from pathlib import Path

import pytest
import torch

from aklr_amd import schema as S
from aklr_amd.schema import __main__ as cli
from aklr_amd.schema import audit, build, text

REF = Path("/root/reference/aklr")
needs_ref = pytest.mark.skipif(not REF.is_dir(), reason="the reference checkout is not here")


def _reference_schemas():
    for p in sorted(REF.rglob("impls/*/*/*.json")):
        yield p, json.loads(p.read_text(encoding="utf-8"))


# ---------------------------------------------------------------------------------------------
# text and uuid
@needs_ref
def test_text_and_uuid_reproduce_every_reference_schema_file():
    n = 0
    for p, s in _reference_schemas():
        assert text.json_file_text(s) == p.read_text(encoding="utf-8"), p
        assert text.schema_uuid(s) == p.stem, p
        assert p.parent.parent.name == s["kernel"]["language"] and p.parent.name == s["name"]
        n += 1
    assert n > 100


def test_json_file_text_known_answer():
    obj = {"b": [1, 2.5], "a": {"x": ["s", 1], "é": None, "e": {}}, "c": []}
    assert text.json_file_text(obj) == (
        '{\n  "b": [1, 2.5],\n  "a": {\n    "x": [\n      "s",\n      1\n    ],\n    "é": null,\n    "e": {}\n'
        '  },\n  "c": []\n}\n')


def _definition(contract_id="gemm_a8w8_blockwise_scaled@1.0", variant="b_shuffled", attrs=None):
    """A definition as export writes one (sources empty), with made-up axes and descriptions."""
    return {
        "schema_version": 5,
        "name": f"{contract_id.split('@')[0]}_{variant}_test",
        "contract_id": contract_id,
        "description": "made up for the test",
        "op_type": "gemm" if "gemm" in contract_id else ("quant" if "quant" in contract_id else "deepseek_v2"),
        "axes": {"m": {"type": "var", "description": "rows"}},
        "attrs": dict(attrs or {}),
        "inputs": {"a": {"shape": ["m", 64], "dtype": "float8_e4m3fn", "description": "x"}},
        "outputs": {"out": {"shape": ["m", 64], "dtype": "bfloat16", "description": "y"}},
        "workloads": [{"axes": {"m": 256}}, {"axes": {"m": 1}, "accuracy": "passed", "speedup": 1.2,
                                              "microseconds": 3.0}],
        "layout_variants": {"by_name": {variant: {"detect_facts": []}}},
        "compare": {"max_violation_fraction": 0.0, "determinism": "bounded", "element_order": "fixed"},
        "kernel": {"language": "flydsl", "targets": [{"arch": "gfx950", "hardware": "MI355X"}],
                   "entry_point": "kernel.py::run", "sources": []},
    }


def test_uuid_moves_with_authored_content_only():
    s = S.fill(_definition())
    u = text.schema_uuid(s)
    measured = copy.deepcopy(s)
    measured["workloads"][0].update(accuracy="passed", speedup=1.5, microseconds=9.0)
    measured["workloads"].reverse()
    measured["description"] = "other prose"  # not authored: export writes it
    assert text.schema_uuid(measured) == u
    for change in (lambda t: t["kernel"].update(author="someone"),
                   lambda t: t["kernel"]["sources"][0].update(content=t["kernel"]["sources"][0]["content"] + "\n"),
                   lambda t: t["workloads"][0].update(scalars={"beta": 0.0}),
                   lambda t: t.update(name="other")):
        t = copy.deepcopy(s)
        change(t)
        assert text.schema_uuid(t) != u


# ---------------------------------------------------------------------------------------------
# call keys
_MDEF = re.compile(r'm\.def\(\s*((?:"[^"]*"\s*)+),')


def _entry_signature(source: str) -> str:
    m = _MDEF.search(source)
    return "".join(re.findall(r'"([^"]*)"', m.group(1)))


@pytest.mark.parametrize("contract_id", sorted(S.CONTRACTS))
def test_each_entry_registers_the_call_keys(contract_id):
    c = S.CONTRACTS[contract_id]
    sig = _entry_signature((S.ENTRIES / c.entry).read_text())
    op_schema = torch._C.parse_schema(sig)
    assert build.op_schema_errors(op_schema, c.call_keys, c.mutable) == []
    assert [a.name for a in op_schema.arguments] == list(c.call_keys)  # in api order, as the reference's own


def _reference_call_keys(s):
    """(argument names, written names) of a committed kernel's entry."""
    entry_file, _, symbol = s["kernel"]["entry_point"].partition("::")
    src = next(x["content"] for x in s["kernel"]["sources"] if x["path"] == entry_file)
    if entry_file.endswith(".hip"):
        op_schema = torch._C.parse_schema(_entry_signature(src))
        return ({a.name for a in op_schema.arguments},
                {a.name for a in op_schema.arguments if a.alias_info is not None and a.alias_info.is_write})
    fn = next(n for n in ast.parse(src).body if isinstance(n, ast.FunctionDef) and n.name == symbol)
    return {a.arg for a in fn.args.kwonlyargs}, None


@needs_ref
def test_call_keys_are_the_reference_kernels():
    seen = set()
    for _, s in _reference_schemas():
        c = S.CONTRACTS.get(s["contract_id"])
        if c is None or not s["kernel"]["sources"]:
            continue
        names, writes = _reference_call_keys(s)
        assert names == set(c.call_keys), s["name"]
        assert set(c.mutable) == set(s["outputs"]), s["name"]
        if writes is not None:
            assert writes == set(c.mutable), s["name"]
        seen.add(s["contract_id"])
    assert seen == set(S.CONTRACTS) - {"gemm_a4w4_mxfp4@1.0"}
    api = ast.parse((REF / "ops" / "gemm" / "api.py").read_text())
    fn = next(n for n in api.body if isinstance(n, ast.FunctionDef) and n.name == "gemm_a4w4_mxfp4")
    params = {a.arg for a in fn.args.args + fn.args.kwonlyargs}
    assert params == set(S.CONTRACTS["gemm_a4w4_mxfp4@1.0"].call_keys)


# ---------------------------------------------------------------------------------------------
# audit
@needs_ref
def test_reference_hip_kernels_pass_the_audit():
    n = 0
    for p, s in _reference_schemas():
        if s["kernel"]["language"] == "hip" and s["kernel"]["sources"]:
            assert audit.findings(s["kernel"]) == [], p
            n += 1
    assert n >= 5


def _kernel(contract_id="gemm_a8w8_blockwise_scaled@1.0", variant="b_shuffled"):
    return S.fill(_definition(contract_id, variant))["kernel"]


@pytest.mark.parametrize("contract_id", sorted(S.CONTRACTS))
def test_every_packaged_kernel_passes(contract_id):
    for variant in S.CONTRACTS[contract_id].variants:
        assert audit.findings(_kernel(contract_id, variant)) == []


def _edit(kernel, path, fn):
    k = copy.deepcopy(kernel)
    src = next(s for s in k["sources"] if s["path"] == path)
    src["content"] = fn(src["content"])
    return k


def _rules(kernel):
    return {f[0] for f in audit.findings(kernel)}


_BODY = "aklr_amd/csrc/quant.hip"


@pytest.mark.parametrize("rule,path,edit", [
    ("SH0", _BODY, lambda t: t + "/* left open\n"),
    ("SH0", _BODY, lambda t: t + 'const char* s = "open\n'),
    ("SH1", "kernel.hip", lambda t: t + "TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, n) {}\n"),
    ("SH1", _BODY, lambda t: t + "TORCH_LIBRARY(other, m) {}\n"),
    ("SH1", _BODY, lambda t: t + "PYBIND11_MODULE(x, m) {}\n"),
    ("SH2", _BODY, lambda t: "#include <mutex>\n" + t),
    ("SH2", _BODY, lambda t: "#include <stdint.h>\n" + t),
    ("SH2", _BODY, lambda t: '#include "absent.h"\n' + t),
    ("SH3", _BODY, lambda t: t + "void f(void** p) { hipMalloc(p, 16); }\n"),
    ("SH3", _BODY, lambda t: t + "void f(void* p) { hipMemset(p, 0, 16); }\n"),
    ("SH3", _BODY, lambda t: t + "void f(void* d, void* s) { hipMemcpyDtoD(d, s, 16); }\n"),
    ("SH3", _BODY, lambda t: t + "void f() { hipDeviceSynchronize(); }\n"),
    # the rule reads names, not calls: every copy-kind name (hipMemcpyKind, hipMemcpyDeviceToDevice) is one
    ("SH3", _BODY, lambda t: t + "int kind = static_cast<int>(hipMemcpyDeviceToDevice);\n"),
    ("SH3", _BODY, lambda t: t + 'void f() { printf("x"); }\n'),
    ("SH3", _BODY, lambda t: t + "void f(void** p) { cudaMalloc(p, 16); }\n"),
    ("SH3", _BODY, lambda t: t + 'const char* f() { return getenv("X"); }\n'),
    ("SH4", _BODY, lambda t: t + "static int calls = 0;\n"),
    ("SH4", _BODY, lambda t: t + "__device__ int counter;\n"),
    ("SH4", _BODY, lambda t: t + "void f() { static int n; }\n"),
    ("SH4", _BODY, lambda t: t + "thread_local int n = 1;\n"),
    ("SH5", "kernel.hip", lambda t: "#include \"entry.h\"\n" + t),
    ("source", _BODY, lambda t: t.replace("\n", "\n\t", 1)),
    ("source", _BODY, lambda t: t.rstrip("\n")),
    ("source", _BODY, lambda t: t + "\n"),
    ("source", _BODY, lambda t: "﻿" + t),
])
def test_each_rule_catches_its_violation(rule, path, edit):
    assert rule in _rules(_edit(_kernel(), path, edit))


@pytest.mark.parametrize("allowed", [
    "const void* copy_entry() { return reinterpret_cast<const void*>(&hipMemcpyAsync); }\n",
    "void f(void* p, hipStream_t st) { hipMemsetAsync(p, 0, 16, st); }\n",
    "static const int kA = 1;\nstatic constexpr int kB = 2;\n",
    "static void helper(int x) { (void)static_cast<long>(x); }\n",
    "__device__ __forceinline__ float twice(float x) { return 2.0f * x; }\n",
    "// hipMalloc(p); static int x = 0; printf(\"\")\n",
    'const char* kName = "hipDeviceSynchronize printf getenv";\n',
    "#include <cstdint>\n#include <ATen/ATen.h>\n#include <hip/hip_fp16.h>\n#include \"common.h\"\n",
    "struct S { static int size() { return 1; } };\n",
])
def test_allowed_lookalikes_pass(allowed):
    assert audit.findings(_edit(_kernel(), _BODY, lambda t: t + allowed)) == []


def test_kernel_section_rules():
    k = _kernel()
    assert _rules({**k, "requires": {}}) == {"kernel"}
    assert "kernel" in _rules({**k, "entry_point": "kernel.py::run"})
    assert "kernel" in _rules({**k, "sources": list(reversed(k["sources"]))})
    bad = copy.deepcopy(k)
    bad["sources"].append({"path": "x-y/z.h", "content": "// z\n"})
    bad["sources"].sort(key=lambda s: s["path"])
    assert "source" in _rules(bad)


# ---------------------------------------------------------------------------------------------
# fill
def _served(s) -> bool:
    c = S.CONTRACTS.get(s["contract_id"])
    if c is None:
        return False
    variant = next(iter(s["layout_variants"]["by_name"]))
    return variant in c.variants and all(s["attrs"].get(a, v[0]) in v for a, v in c.attrs_served.items())


@needs_ref
def test_fill_every_reference_definition_of_this_path(tmp_path):
    filled = {}
    for p, s in _reference_schemas():
        if not _served(s):
            continue
        f = S.fill(s)
        rest = lambda x: {k: v for k, v in x.items() if k not in ("kernel", "workloads")}
        assert rest(f) == rest(s)
        assert [w for w in f["workloads"]] == [{k: v for k, v in w.items() if k not in S.MEASUREMENTS}
                                              for w in s["workloads"]]
        assert f["kernel"]["targets"] == s["kernel"]["targets"]
        assert list(f["kernel"]) == ["language", "targets", "requires", "author", "entry_point", "sources"]
        out = S.write(f, tmp_path)
        assert S.check(out) == [], out
        assert out.relative_to(tmp_path).parts[:3] == (s["op_type"], "impls", "hip")
        filled[s["contract_id"]] = filled.get(s["contract_id"], 0) + 1
    assert set(filled) >= {"gemm_a8w8_blockwise_scaled@1.0", "per_group_quant_fp8@1.0",
                           "per_group_quant_mxfp8@1.0", "deepseek_v2_fp8_moe@1.0"}


def test_fill_refuses_what_it_has_no_kernel_for():
    with pytest.raises(S.PackagingError, match="no kernel here for"):
        S.fill(_definition("gemm@1.0", "row_major"))
    with pytest.raises(S.PackagingError, match="layout variant"):
        S.fill(_definition(variant="b_preshuffled_32x32"))
    with pytest.raises(S.PackagingError, match="trans_b"):
        S.fill(_definition("gemm_a4w4_mxfp4@1.0", "row_major", attrs={"trans_b": False}))
    # the FP8 GEMM's row_major kernel takes b as (k, n) too
    assert S.fill(_definition(variant="row_major", attrs={"trans_b": False}))["kernel"]["language"] == "hip"
    with pytest.raises(S.PackagingError, match="scoring_func"):
        S.fill(_definition("deepseek_v2_fp8_moe@1.0", "shuffled_16x16", attrs={"scoring_func": "softmax"}))
    d = _definition()
    d["kernel"]["targets"] = [{"arch": "gfx942"}]
    with pytest.raises(S.PackagingError, match="gfx950"):
        S.fill(d)
    d = _definition()
    d["schema_version"] = 4
    with pytest.raises(S.PackagingError, match="schema_version"):
        S.fill(d)


def test_packaged_sources_are_the_repository_files():
    k = _kernel()
    files = {s["path"]: s["content"] for s in k["sources"]}
    assert files["kernel.hip"] == (S.ENTRIES / "gemm_a8w8_blockwise_scaled.hip").read_text()
    for name in ("common.h", "gemm_a8w8.hip", "quant.hip"):
        assert files[f"aklr_amd/csrc/{name}"] == (S.ROOT / "aklr_amd" / "csrc" / name).read_text()
    header = (S.ROOT / "include" / "aklr_amd.h").read_text()
    assert files["include/aklr_amd.h"] == header.replace("<stddef.h>", "<cstddef>").replace("<stdint.h>", "<cstdint>")
    assert "constexpr bool a_scale_column_major = true;" in files["variant.h"]


def test_cli_fill_then_check(tmp_path, capsys):
    d = tmp_path / "definition.json"
    d.write_text(text.json_file_text(_definition()))
    assert cli.main(["fill", str(d), "--to", str(tmp_path / "out")]) == 0
    written = Path(capsys.readouterr().out.strip())
    assert written.is_file() and cli.main(["check", str(written)]) == 0
    moved = written.with_name("0000000000000000.json")
    written.rename(moved)
    assert cli.main(["check", str(moved)]) == 1


@pytest.mark.parametrize("contract_id,variant", build.TESTED)
def test_built_libraries_register_the_call_keys(contract_id, variant):
    kernel = build.tested_kernel(contract_id, variant)
    if not build.library_path(kernel).exists():
        pytest.skip("packages not built (__graft_entry__.build() builds them)")
    c = S.CONTRACTS[contract_id]
    op = build.load(kernel)
    assert build.op_schema_errors(op.default._schema, c.call_keys, c.mutable) == []


def test_kernel_sources_switch_packed_fp32_off():
    """AKLR builds the packaged sources with -O3 only, so each kernel source must switch packed fp32 VALU
    ops off itself: AKLR_SCALAR_FP32_BEGIN after its last include and AKLR_SCALAR_FP32_END as its last
    line (common.h wraps its own functions the same way)."""
    from pathlib import Path

    csrc = Path(__file__).resolve().parent.parent / "aklr_amd" / "csrc"
    files = sorted(csrc.glob("*.hip")) + [csrc / "common.h"]
    assert len(files) >= 7
    for f in files:
        lines = [ln for ln in f.read_text().splitlines() if ln.strip()]
        begin = [i for i, ln in enumerate(lines) if ln == "AKLR_SCALAR_FP32_BEGIN"]
        end = [i for i, ln in enumerate(lines) if ln == "AKLR_SCALAR_FP32_END"]
        assert len(begin) == 1 and len(end) == 1, f"{f.name}: one BEGIN and one END"
        last_include = max(i for i, ln in enumerate(lines) if ln.startswith("#include"))
        assert begin[0] > last_include, f"{f.name}: BEGIN comes after the includes"
        if f.suffix == ".hip":
            assert end[0] == len(lines) - 1, f"{f.name}: END is the last line"
