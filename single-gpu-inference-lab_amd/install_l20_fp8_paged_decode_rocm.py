#!/usr/bin/env python3
"""Install (or remove) the gated MI355X paged FP8 decode path in vLLM's ROCm backend.

The ROCm counterpart of ``integrations/vllm/install_l20_fp8_paged_decode.py``
(paths relative to the reference repo root), which patches the CUDA FlashInfer
backend.  Here the patch point is the ``unified_attention(`` call of vLLM's
Triton attention backend (``vllm/v1/attention/backends/triton_attn.py``, the
ROCm backend whose KV cache is NHD ``[num_blocks, 16, num_kv_heads,
head_size]``).  The installer

* keeps a backup of the backend file beside it (``.py.l20-fp8-paged-backup``);
* writes ``vllm/v1/attention/ops/l20_rocm_fp8_decode.py``, a shim that puts this
  package on ``sys.path`` and re-exports ``l20_fp8_paged_decode_or_none`` from
  ``l20_vllm_rocm_hook`` (gates: VLLM_ENABLE_L20_FP8_PAGED_DECODE,
  VLLM_L20_FP8_PAGED_FORCE, VLLM_L20_FP8_PAGED_TRACE);
* inserts the gated call before ``unified_attention(``, once (re-running is a
  no-op); ``--uninstall`` restores the backup and removes the shim.

Usage: ``python install_l20_fp8_paged_decode_rocm.py [--vllm-source-dir DIR] [--uninstall]``
"""

from __future__ import annotations

import argparse
import importlib.util
import shutil
from pathlib import Path
from typing import Optional

HERE = Path(__file__).resolve().parent
BACKEND = Path("v1/attention/backends/triton_attn.py")
SHIM = Path("v1/attention/ops/l20_rocm_fp8_decode.py")
BACKUP_SUFFIX = ".py.l20-fp8-paged-backup"

PATCH_ANCHOR = """        unified_attention(
            q=query[:num_actual_tokens],
"""
PATCH_CALL = """        from vllm.v1.attention.ops.l20_rocm_fp8_decode import (
            l20_fp8_paged_decode_or_none,
        )

        if l20_fp8_paged_decode_or_none(self, layer, query, key_cache,
                                        value_cache, output, attn_metadata,
                                        num_actual_tokens,
                                        output_scale=locals().get("output_scale")):
            return output

"""

SHIM_TEXT = '''"""Written by install_l20_fp8_paged_decode_rocm.py: the MI355X paged FP8 decode hook."""

import sys

_PACKAGE = {package!r}
if _PACKAGE not in sys.path:
    sys.path.insert(0, _PACKAGE)

from l20_vllm_rocm_hook import l20_fp8_paged_decode_or_none  # noqa: E402,F401
'''


def replace_once(source: str, old: str, new: str, label: str) -> str:
    """Insert ``new`` in place of ``old`` unless it is already there."""
    if new in source:
        return source
    if old not in source:
        raise RuntimeError(f"cannot find patch point: {label}")
    return source.replace(old, new, 1)


def patch_source(source: str) -> str:
    """The backend source with the gated call inserted before ``unified_attention(``."""
    return replace_once(source, PATCH_ANCHOR, PATCH_CALL + PATCH_ANCHOR, "Triton unified_attention call")


def find_vllm_package(source_dir: Optional[str]) -> Path:
    candidates = []
    if source_dir:
        candidates.append(Path(source_dir).expanduser().resolve() / "vllm")
    spec = importlib.util.find_spec("vllm") if source_dir is None else None
    if spec is not None and spec.origin:
        candidates.append(Path(spec.origin).resolve().parent)
    candidates.append(Path.cwd() / "vllm")
    for candidate in candidates:
        if (candidate / BACKEND).exists():
            return candidate
    raise RuntimeError("cannot find vLLM source package")


def install(package: Path) -> None:
    backend = package / BACKEND
    backup = backend.with_suffix(BACKUP_SUFFIX)
    if not backup.exists():
        shutil.copy2(backend, backup)
    shim = package / SHIM
    shim.parent.mkdir(parents=True, exist_ok=True)
    shim.write_text(SHIM_TEXT.format(package=str(HERE)), encoding="utf-8")
    backend.write_text(patch_source(backend.read_text(encoding="utf-8")), encoding="utf-8")


def uninstall(package: Path) -> None:
    backend = package / BACKEND
    backup = backend.with_suffix(BACKUP_SUFFIX)
    if backup.exists():
        shutil.copy2(backup, backend)
        backup.unlink()
    shim = package / SHIM
    if shim.exists():
        shim.unlink()


def main(argv: Optional[list] = None) -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--vllm-source-dir")
    parser.add_argument("--uninstall", action="store_true")
    args = parser.parse_args(argv)
    package = find_vllm_package(args.vllm_source_dir)
    if args.uninstall:
        uninstall(package)
    else:
        install(package)
    print(package)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
