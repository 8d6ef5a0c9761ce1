"""AKLR schema packaging: this library's kernels as HIP kernel schema files that an unmodified AKLR loads,
audits, builds and benchmarks (aklr/ops/README.md:35-62 workflow steps 3-4, :183-286 the HIP kernel ABI).

AKLR serves a kernel from a schema file ``<op>/impls/hip/<name>/<uuid>.json``. ``python -m aklr
export`` writes one per scenario with ``"sources": []`` (a definition); its author fills
``kernel.sources``, ``requires`` and ``author``, and renames the file to the uuid of what was written.
``fill(definition)`` does exactly that for the contracts of this path:

- ``kernel.sources``: a ``kernel.hip`` entry that registers ``run(<the contract's call keys>) -> ()``
  in ``TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, m)`` and calls this library's C ABI, ``entry.h``,
  ``variant.h`` (the schema's layout variant as constants), this library's kernel sources and
  ``include/aklr_amd.h``, at their repository paths so that their includes resolve;
- ``kernel.language`` ``hip`` and ``entry_point`` ``kernel.hip::run`` (what ``export --language hip``
  writes; a definition exported for another language is rewritten to them), ``targets`` as exported;
- ``requires`` ``{"hip": ">=<the HIP torch was built with, major.minor>"}`` and ``author``;
- the workloads' ``accuracy``, ``speedup`` and ``microseconds`` are dropped (only AKLR's CI writes them).

The filled text is checked against the rules an unmodified AKLR applies (``audit``) before it is
returned; ``check(path)`` re-checks a written file. Everything else in the file is the definition's,
unchanged: AKLR's ``export check`` requires that.
"""
from __future__ import annotations

import copy
import json
from dataclasses import dataclass, field
from pathlib import Path, PurePosixPath
from typing import Any, Mapping

from . import audit, text

__all__ = ["CONTRACTS", "PackagingError", "check", "fill", "kernel_sources", "write"]

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent.parent
ENTRIES = PKG / "entries"
ENTRY_POINT = "kernel.hip::run"
REQUIRES = {"hip": ">=7.0"}  # torch.version.hip of the toolchain these kernels were developed on
AUTHOR = "aklr_amd"
MEASUREMENTS = ("accuracy", "speedup", "microseconds")


class PackagingError(ValueError):
    """A definition this library has no kernel for, or a filled file AKLR would reject."""


@dataclass(frozen=True)
class Contract:
    entry: str  # file under entries/, shipped as kernel.hip
    csrc: tuple[str, ...]  # kernel sources under aklr_amd/csrc
    variants: Mapping[str, Mapping[str, bool] | None]  # layout variant -> variant.h constants (None: no header)
    # the call keys of the contract's kernel entry, in api order (aklr/core/contract/op.py:511-558)
    call_keys: tuple[str, ...]
    mutable: tuple[str, ...]
    attrs_served: Mapping[str, tuple] = field(default_factory=dict)  # attrs whose values the kernels take


_QUANT_KEYS = ("x", "quantized", "scales")
CONTRACTS: dict[str, Contract] = {
    # aklr/ops/quant/contract.py:17-51
    "per_group_quant_fp8@1.0": Contract("per_group_quant_fp8.hip", ("quant.hip",), {"row_major": None},
                                        _QUANT_KEYS, ("quantized", "scales")),
    # aklr/ops/quant/contract.py:54-75
    "per_group_quant_mxfp8@1.0": Contract("per_group_quant_mxfp8.hip", ("quant.hip",), {"row_major": None},
                                          _QUANT_KEYS, ("quantized", "scales")),
    # aklr/ops/gemm/contract.py:211-308
    "gemm_a8w8_blockwise_scaled@1.0": Contract(
        "gemm_a8w8_blockwise_scaled.hip", ("gemm_a8w8.hip", "quant.hip"),
        {
            "row_major": {"b_preshuffled": False, "a_scale_column_major": False},
            "b_shuffled": {"b_preshuffled": True, "a_scale_column_major": True},
            "b_shuffled_row_major_a_scale": {"b_preshuffled": True, "a_scale_column_major": False},
        },
        ("a", "b", "a_scale", "b_scale", "scale_major_mode", "trans_b", "operand_format", "bias", "out_dtype", "out"),
        ("out",), {"trans_b": (True, False)}),  # trans_b = False: row_major only (contract.py:242-246)
    # aklr/ops/gemm/contract.py:315-390
    "gemm_a4w4_mxfp4@1.0": Contract(
        "gemm_a4w4_mxfp4.hip", ("gemm_a4w4.hip", "quant.hip"),
        {"row_major": {"shuffled": False}, "b_shuffled": {"shuffled": True}},
        ("a", "b", "a_scale", "b_scale", "trans_b", "operand_format", "alpha", "beta", "bias", "out_dtype", "out"),
        ("out",), {"trans_b": (True,)}),
    # aklr/plugins/sglang/models/deepseek_v2/contract.py:188-320
    "deepseek_v2_fp8_moe@1.0": Contract(
        "deepseek_v2_fp8_moe.hip", ("moe_fp8.hip", "quant.hip"),
        {"row_major": {"weights_preshuffled": False}, "shuffled_16x16": {"weights_preshuffled": True}},
        ("hidden_states", "router_weight", "correction_bias", "w1", "w1_scale", "w2", "w2_scale", "topk",
         "num_expert_group", "topk_group", "renormalize", "scoring_func", "routed_scaling_factor", "out_dtype",
         "out"),
        ("out",), {"scoring_func": ("sigmoid",)}),
}


def _read(path: Path) -> str:
    return path.read_text(encoding="utf-8")


def _variant_header(variant: str, constants: Mapping[str, bool]) -> str:
    lines = [f"// Layout variant of this kernel's schema: {variant}.", "#pragma once", "", "namespace aklr_variant {"]
    lines += [f"constexpr bool {name} = {'true' if value else 'false'};" for name, value in constants.items()]
    lines += ["}  // namespace aklr_variant", ""]
    return "\n".join(lines)


def _c_header_for_cxx() -> str:
    """include/aklr_amd.h as the packaged C++ sources include it: its two C standard headers under
    their C++ names, the only spellings AKLR's include rule admits (the declarations are unchanged)."""
    header = _read(ROOT / "include" / "aklr_amd.h")
    c_includes = "#include <stddef.h>\n#include <stdint.h>\n"
    if c_includes not in header:
        raise PackagingError("include/aklr_amd.h no longer includes <stddef.h> and <stdint.h> as expected")
    return header.replace(c_includes, "#include <cstddef>\n#include <cstdint>\n", 1)


def kernel_sources(contract_id: str, variant: str) -> list[dict[str, str]]:
    """The ``kernel.sources`` of ``contract_id`` at layout ``variant``, sorted by path."""
    contract = _contract(contract_id)
    if variant not in contract.variants:
        raise PackagingError(f"{contract_id}: no kernel here for layout variant {variant!r}")
    files = {
        "kernel.hip": _read(ENTRIES / contract.entry),
        "entry.h": _read(ENTRIES / "entry.h"),
        "include/aklr_amd.h": _c_header_for_cxx(),
        "aklr_amd/csrc/common.h": _read(ROOT / "aklr_amd" / "csrc" / "common.h"),
    }
    for name in contract.csrc:
        files[f"aklr_amd/csrc/{name}"] = _read(ROOT / "aklr_amd" / "csrc" / name)
    constants = contract.variants[variant]
    if constants is not None:
        files["variant.h"] = _variant_header(variant, constants)
    return [{"path": p, "content": files[p]} for p in sorted(files)]


def _contract(contract_id: str) -> Contract:
    try:
        return CONTRACTS[contract_id]
    except KeyError:
        raise PackagingError(f"no kernel here for {contract_id}; this library packages {sorted(CONTRACTS)}") from None


def _variant_of(schema: Mapping[str, Any]) -> str:
    by_name = schema.get("layout_variants", {}).get("by_name", {})
    if len(by_name) != 1:
        raise PackagingError(f"{schema.get('name')}: a schema holds one layout variant, not {sorted(by_name)}")
    return next(iter(by_name))


def _targets_gfx950(targets) -> bool:
    return any(t.get("arch") == "gfx950" or (t.get("arch") is None and t.get("hardware") == "MI355X") for t in targets)


def fill(definition: Mapping[str, Any], *, author: str = AUTHOR) -> dict[str, Any]:
    """The schema ``definition`` (an export's, or a committed file's) with this library's kernel."""
    schema = copy.deepcopy(dict(definition))
    if schema.get("schema_version") != 5:
        raise PackagingError(f"{schema.get('name')}: schema_version {schema.get('schema_version')!r}, expected 5")
    contract = _contract(schema.get("contract_id"))
    variant = _variant_of(schema)
    for attr, served in contract.attrs_served.items():
        if attr in schema.get("attrs", {}) and schema["attrs"][attr] not in served:
            raise PackagingError(f"{schema['name']}: no kernel here for {attr}={schema['attrs'][attr]!r}")
    targets = schema.get("kernel", {}).get("targets") or []
    if not _targets_gfx950(targets):
        raise PackagingError(f"{schema['name']}: targets {targets} name no gfx950 / MI355X; the kernels are gfx950 only")
    kernel: dict[str, Any] = {"language": "hip", "targets": targets}
    if REQUIRES:
        kernel["requires"] = dict(REQUIRES)
    if author:
        kernel["author"] = author
    kernel["entry_point"] = ENTRY_POINT
    kernel["sources"] = kernel_sources(schema["contract_id"], variant)
    schema["kernel"] = kernel
    schema["workloads"] = [{k: v for k, v in w.items() if k not in MEASUREMENTS} for w in schema.get("workloads", [])]
    problems = audit.findings(kernel)
    if problems:
        raise PackagingError("AKLR would reject the kernel:\n" + "\n".join(f"  {r} {p}:{n} {w}" for r, p, n, w in problems))
    return schema


def path_of(schema: Mapping[str, Any]) -> PurePosixPath:
    """Where the file goes below the op family's parent directory: ``<op>/impls/hip/<name>/<uuid>.json``."""
    return PurePosixPath(schema["op_type"]) / text.relative_path(schema)


def write(schema: Mapping[str, Any], to: Path) -> Path:
    path = Path(to) / path_of(schema)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(text.json_file_text(schema), encoding="utf-8")
    return path


def check(path: Path) -> list[str]:
    """What an unmodified AKLR would reject in the schema file at ``path``: its text not in canonical
    form, its name not its uuid, or its kernel failing the source rules and SH0-SH5."""
    raw = Path(path).read_text(encoding="utf-8")
    schema = json.loads(raw)
    problems = []
    if text.json_file_text(schema) != raw:
        problems.append("text is not in the canonical form")
    if Path(path).stem != text.schema_uuid(schema):
        problems.append(f"named {Path(path).stem}, its uuid is {text.schema_uuid(schema)}")
    if Path(path).parent.name != schema.get("name") or Path(path).parent.parent.name != schema["kernel"]["language"]:
        problems.append("not under impls/<language>/<name>/")
    problems += [f"{r} {p}:{n} {w}" for r, p, n, w in audit.findings(schema["kernel"])]
    return problems
