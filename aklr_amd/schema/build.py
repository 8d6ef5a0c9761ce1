"""Builds a filled schema's kernel the way AKLR's HIP builder does (aklr/core/jit/hip_extension.py:54-104,
aklr/core/runtime/builder/builder.py:256-298): the sources written out at their paths,
``torch.utils.cpp_extension.load`` of the ``.hip`` files with the source root on the include path,
``-O3`` for the arch alone, the extension (and op namespace) named ``aklr_hip_<16 hex digits of the
content hash>``, loaded with ``torch.ops.load_library``. No flag is added: the sources themselves switch
packed fp32 VALU ops off (AKLR_SCALAR_FP32_BEGIN/END in csrc/common.h), so the library built here is
the one an unmodified AKLR builds. The libraries go in-tree under ``aklr_amd/schema/_built/`` so that a
GPU run loads what was built here, and ``op_schema_errors`` restates the builder's check of the op it
registers (builder.py:309-323)."""
from __future__ import annotations

import os
import shutil
from pathlib import Path
from typing import Any, Collection, Mapping

from . import text

BUILT = Path(__file__).resolve().parent / "_built"
ARCH = "gfx950"
FLAGS = ["-O3"]


def library_path(kernel: Mapping[str, Any], root: Path = BUILT) -> Path:
    name = text.extension_name(kernel)
    return root / name / f"{name}.so"


def build(kernel: Mapping[str, Any], root: Path = BUILT) -> Path:
    """Compile ``kernel``'s sources into ``root/<name>/<name>.so`` (every time); returns its path."""
    from torch.utils import cpp_extension

    name = text.extension_name(kernel)
    build_dir = root / name
    if build_dir.exists():
        shutil.rmtree(build_dir)
    src = build_dir / "src"
    for s in kernel["sources"]:
        (src / s["path"]).parent.mkdir(parents=True, exist_ok=True)
        (src / s["path"]).write_text(s["content"], encoding="utf-8")
    previous = os.environ.get("PYTORCH_ROCM_ARCH")
    os.environ["PYTORCH_ROCM_ARCH"] = ARCH
    try:
        cpp_extension.load(
            name=name,
            sources=[str(src / s["path"]) for s in sorted(kernel["sources"], key=lambda s: s["path"])
                     if s["path"].endswith(".hip")],
            extra_include_paths=[str(src)],
            extra_cuda_cflags=list(FLAGS),
            build_directory=str(build_dir),
            is_python_module=False,
        )
    finally:
        if previous is None:
            del os.environ["PYTORCH_ROCM_ARCH"]
        else:
            os.environ["PYTORCH_ROCM_ARCH"] = previous
    return build_dir / f"{name}.so"


def load(kernel: Mapping[str, Any], root: Path = BUILT):
    """The registered op ``torch.ops.<name>.run`` of the built library (which must exist)."""
    import torch

    path = library_path(kernel, root)
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build() (or aklr_amd.schema.build.build)")
    name = text.extension_name(kernel)
    if not hasattr(getattr(torch.ops, name), "run"):
        torch.ops.load_library(str(path))
    return getattr(torch.ops, name).run


def op_schema_errors(op_schema, call_keys: Collection[str], mutable_tensors: Collection[str]) -> list[str]:
    """Why AKLR's HIP builder would refuse the registered op: its arguments are not exactly the call
    keys, it does not write exactly the mutable tensors (each a ``Tensor(a!)``), or it returns
    something."""
    names = [a.name for a in op_schema.arguments]
    errors = []
    if sorted(names) != sorted(call_keys):
        errors.append(f"takes {names}, not the call keys {list(call_keys)}")
    writes = {a.name for a in op_schema.arguments if a.alias_info is not None and a.alias_info.is_write}
    if writes != set(mutable_tensors):
        errors.append(f"writes {sorted(writes)}, not {sorted(mutable_tensors)}")
    if op_schema.returns:
        errors.append(f"returns {op_schema.returns}, not ()")
    return errors


# The packages the GPU parity test loads: one per contract at its aiter layout, and the FP8 GEMM's
# row-major variant too (K-major scales, bias).
TESTED = (
    ("per_group_quant_fp8@1.0", "row_major"),
    ("per_group_quant_mxfp8@1.0", "row_major"),
    ("gemm_a8w8_blockwise_scaled@1.0", "b_shuffled"),
    ("gemm_a8w8_blockwise_scaled@1.0", "row_major"),
    ("gemm_a4w4_mxfp4@1.0", "b_shuffled"),
    ("deepseek_v2_fp8_moe@1.0", "shuffled_16x16"),
)


def tested_kernel(contract_id: str, variant: str) -> dict[str, Any]:
    """The kernel section ``fill`` writes for ``contract_id`` at ``variant`` (targets aside, which do not
    enter the build)."""
    from . import ENTRY_POINT, REQUIRES, kernel_sources

    return {"language": "hip", "targets": [{"arch": ARCH}], "requires": dict(REQUIRES), "entry_point": ENTRY_POINT,
            "sources": kernel_sources(contract_id, variant)}


def _build_kept(kernel: Mapping[str, Any]) -> str:
    """Build, then keep the library alone: objects and the written sources stay out of the snapshot a
    GPU run receives."""
    path = build(kernel)
    for item in path.parent.iterdir():
        if item != path:
            shutil.rmtree(item) if item.is_dir() else item.unlink()
    return str(path)


def build_tested(workers: int = 3) -> list[Path]:
    """Build every package of ``TESTED`` (separate processes, ``workers`` at once) and remove
    libraries of sources that changed since."""
    import concurrent.futures
    import multiprocessing

    kernels = [tested_kernel(c, v) for c, v in TESTED]
    keep = {text.extension_name(k) for k in kernels}
    if BUILT.exists():
        for stale in BUILT.iterdir():
            if stale.name not in keep:
                shutil.rmtree(stale) if stale.is_dir() else stale.unlink()
    ctx = multiprocessing.get_context("spawn")
    with concurrent.futures.ProcessPoolExecutor(max_workers=workers, mp_context=ctx) as pool:
        return [Path(p) for p in pool.map(_build_kept, kernels)]
