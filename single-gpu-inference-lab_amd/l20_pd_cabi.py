"""ctypes binding of the C ABI in ``include/l20_paged_decode.h`` and ``include/l20_kv_write.h``.

Loads ``libl20_paged_decode_hip.so`` from beside this file and mirrors the
``l20_pd_fp8_args`` struct field by field.  ``args_from_tensors`` fills the
struct from torch tensors (device pointers, sizes, strides) so that tests and
benchmarks can call the library without the torch dispatcher in between.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).with_name("libl20_paged_decode_hip.so")

L20_PD_BF16, L20_PD_FP16, L20_PD_FP32 = 0, 1, 2
L20_PD_OK, L20_PD_EINVAL, L20_PD_ELAUNCH = 0, 1, 2
L20_PD_KV_FP8_E4M3, L20_PD_KV_FP16, L20_PD_KV_BF16, L20_PD_KV_FP8_E5M2 = 0, 1, 2, 3
L20_PD_DEVERR_PREFIX_WAIT, L20_PD_DEVERR_ACK_WAIT, L20_PD_DEVERR_PUBLISH_WAIT = 1, 2, 4
L20_PD_DEVERR_QUEUE_SHARED = 32
ABI_VERSION = 4

# Every extern "C" symbol declared in include/*.h.
EXPORTED = (
    "l20_pd_abi_version",
    "l20_pd_last_error",
    "l20_pd_num_splits",
    "l20_pd_fp8_e4m3_check",
    "l20_pd_fp8_e4m3_split_out",
    "l20_pd_fp8_e4m3_split_out_noalloc",
    "l20_pd_device_errors",
    "l20_pd_set_spin_limit",
    "l20_pd_set_queue_counters",
    "l20_pd_single_launch",
    "l20_pd_split_out",
    "l20_pd_fp8_e4m3_partial",
    "l20_pd_fp8_e4m3_merge",
    "l20_pd_default_split_size",
    "l20_pd_fp8_e4m3_dequant_f32",
    "l20_pd_fp8_e4m3_dequant_bf16",
    "l20_pd_stream_read",
    "l20_pd_stream_copy",
    "l20_pd_kv_write_check",
    "l20_pd_rope_and_cache",
    "l20_pd_kv_fp8_scales",
    "l20_pd_tree_suffix_check",
    "l20_pd_tree_suffix_merge",
)

_i32, _i64, _f32, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class L20PdFp8Args(ctypes.Structure):
    _fields_ = [
        ("query", _vp), ("query_dtype", _i32), ("q_stride_row", _i64), ("q_stride_head", _i64),
        ("key_cache", _vp), ("k_stride_page", _i64), ("k_stride_token", _i64), ("k_stride_head", _i64),
        ("value_cache", _vp), ("v_stride_page", _i64), ("v_stride_token", _i64), ("v_stride_head", _i64),
        ("num_pages", _i64), ("page_size", _i32),
        ("block_table", _vp), ("bt_stride_row", _i64), ("bt_max_pages", _i32),
        ("seq_lens", _vp),
        ("partial_output", _vp), ("partial_dtype", _i32),
        ("po_stride_row", _i64), ("po_stride_head", _i64), ("po_stride_split", _i64),
        ("partial_splits", _i32),
        ("partial_max", _vp), ("pm_stride_row", _i64), ("pm_stride_head", _i64), ("pm_stride_split", _i64),
        ("partial_sum", _vp), ("ps_stride_row", _i64), ("ps_stride_head", _i64), ("ps_stride_split", _i64),
        ("output", _vp), ("o_stride_row", _i64), ("o_stride_head", _i64),
        ("lse", _vp), ("lse_stride_row", _i64), ("lse_stride_head", _i64),
        ("k_scale", _f32), ("v_scale", _f32),
        ("k_scale_per_head", _vp), ("v_scale_per_head", _vp),
        ("softmax_scale", _f32),
        ("batch", _i32), ("q_len", _i32), ("num_q_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("max_seq_len", _i32), ("split_size", _i32),
        ("kv_dtype", _i32), ("page_indptr", _vp),
        ("tree_mask", _vp), ("tree_mask_stride_batch", _i64),
    ]


class L20PdTreeSuffixArgs(ctypes.Structure):
    """Mirror of ``l20_pd_tree_suffix_args`` (include/l20_tree_verify.h)."""

    _fields_ = [
        ("query", _vp), ("q_stride_batch", _i64), ("q_stride_draft", _i64), ("q_stride_head", _i64),
        ("query_dtype", _i32),
        ("suffix_key", _vp), ("sk_stride_batch", _i64), ("sk_stride_draft", _i64), ("sk_stride_head", _i64),
        ("suffix_value", _vp), ("sv_stride_batch", _i64), ("sv_stride_draft", _i64), ("sv_stride_head", _i64),
        ("ancestor_mask", _vp), ("mask_stride_row", _i64), ("mask_stride_col", _i64),
        ("prefix_output", _vp), ("po_stride_batch", _i64), ("po_stride_draft", _i64), ("po_stride_head", _i64),
        ("prefix_dtype", _i32),
        ("prefix_lse", _vp), ("pl_stride_batch", _i64), ("pl_stride_draft", _i64), ("pl_stride_head", _i64),
        ("output", _vp), ("o_stride_batch", _i64), ("o_stride_draft", _i64), ("o_stride_head", _i64),
        ("softmax_scale", _f32),
        ("batch", _i32), ("draft_length", _i32), ("num_q_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
    ]


class L20PdKvWriteArgs(ctypes.Structure):
    """Mirror of ``l20_pd_kv_write_args`` (include/l20_kv_write.h)."""

    _fields_ = [
        ("query", _vp), ("q_stride_token", _i64), ("q_stride_head", _i64), ("num_q_heads", _i32),
        ("key", _vp), ("k_stride_token", _i64), ("k_stride_head", _i64),
        ("value", _vp), ("v_stride_token", _i64), ("v_stride_head", _i64),
        ("dtype", _i32),
        ("positions", _vp), ("cos_sin_cache", _vp), ("cs_stride_position", _i64), ("cs_dtype", _i32),
        ("rotary_dim", _i32), ("is_neox", _i32),
        ("slot_mapping", _vp),
        ("key_cache", _vp), ("kc_stride_page", _i64), ("kc_stride_token", _i64), ("kc_stride_head", _i64),
        ("value_cache", _vp), ("vc_stride_page", _i64), ("vc_stride_token", _i64), ("vc_stride_head", _i64),
        ("num_pages", _i64), ("cache_dtype", _i32),
        ("k_scale", _f32), ("v_scale", _f32), ("k_scale_per_head", _vp), ("v_scale_per_head", _vp),
        ("num_tokens", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
    ]


_lib: Optional[ctypes.CDLL] = None


def load(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load the C ABI library (raises if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    lib_path = Path(path) if path else LIB_PATH
    if not lib_path.exists():
        raise OSError(f"{lib_path} is missing: build it with l20_pd_build.py")
    lib = ctypes.CDLL(str(lib_path))
    lib.l20_pd_abi_version.restype = _i32
    lib.l20_pd_last_error.restype = ctypes.c_char_p
    lib.l20_pd_num_splits.argtypes = [_i32, _i32]
    lib.l20_pd_num_splits.restype = _i32
    args_p = ctypes.POINTER(L20PdFp8Args)
    lib.l20_pd_fp8_e4m3_check.argtypes = [args_p]
    lib.l20_pd_fp8_e4m3_check.restype = _i32
    for name in ("l20_pd_fp8_e4m3_split_out", "l20_pd_fp8_e4m3_split_out_noalloc", "l20_pd_split_out",
                 "l20_pd_fp8_e4m3_partial", "l20_pd_fp8_e4m3_merge"):
        getattr(lib, name).argtypes = [args_p, _vp]
        getattr(lib, name).restype = _i32
    lib.l20_pd_device_errors.argtypes = [_i32]
    lib.l20_pd_device_errors.restype = _i32
    lib.l20_pd_set_spin_limit.argtypes = [ctypes.c_uint32]
    lib.l20_pd_set_spin_limit.restype = _i32
    lib.l20_pd_set_queue_counters.argtypes = [ctypes.c_uint64]
    lib.l20_pd_set_queue_counters.restype = _i32
    lib.l20_pd_single_launch.argtypes = [ctypes.POINTER(L20PdFp8Args)]
    lib.l20_pd_single_launch.restype = _i32
    lib.l20_pd_default_split_size.argtypes = [_i32, _i32, _i32, _i32]
    lib.l20_pd_default_split_size.restype = _i32
    lib.l20_pd_fp8_e4m3_dequant_f32.argtypes = [_vp, _vp, _i64, _f32, _vp]
    lib.l20_pd_fp8_e4m3_dequant_f32.restype = _i32
    lib.l20_pd_fp8_e4m3_dequant_bf16.argtypes = [_vp, _vp, _i64, _vp]
    lib.l20_pd_fp8_e4m3_dequant_bf16.restype = _i32
    lib.l20_pd_stream_read.argtypes = [_vp, _i64, _vp, _i32, _vp]
    lib.l20_pd_stream_read.restype = _i32
    lib.l20_pd_stream_copy.argtypes = [_vp, _vp, _i64, _i32, _vp]
    lib.l20_pd_stream_copy.restype = _i32
    kv_p = ctypes.POINTER(L20PdKvWriteArgs)
    lib.l20_pd_kv_write_check.argtypes = [kv_p]
    lib.l20_pd_kv_write_check.restype = _i32
    lib.l20_pd_rope_and_cache.argtypes = [kv_p, _vp]
    lib.l20_pd_rope_and_cache.restype = _i32
    lib.l20_pd_kv_fp8_scales.argtypes = [kv_p, _vp, _vp, _i32, _vp]
    lib.l20_pd_kv_fp8_scales.restype = _i32
    ts_p = ctypes.POINTER(L20PdTreeSuffixArgs)
    lib.l20_pd_tree_suffix_check.argtypes = [ts_p]
    lib.l20_pd_tree_suffix_check.restype = _i32
    lib.l20_pd_tree_suffix_merge.argtypes = [ts_p, _vp]
    lib.l20_pd_tree_suffix_merge.restype = _i32
    if path is None:
        _lib = lib
    return lib


def last_error(lib: Optional[ctypes.CDLL] = None) -> str:
    return (lib or load()).l20_pd_last_error().decode()


def _dtype_code(t) -> int:
    import torch

    return {torch.bfloat16: L20_PD_BF16, torch.float16: L20_PD_FP16, torch.float32: L20_PD_FP32}[t.dtype]


def _kv_code(t) -> int:
    import torch

    if t.dtype == torch.float16:
        return L20_PD_KV_FP16
    if t.dtype == torch.bfloat16:
        return L20_PD_KV_BF16
    if t.dtype == torch.float8_e5m2:
        return L20_PD_KV_FP8_E5M2
    return L20_PD_KV_FP8_E4M3


def args_from_tensors(query, key_cache, value_cache, block_table, seq_lens, partial_output, partial_max,
                      partial_sum, output, k_scale, v_scale, max_seq_len, split_size, *, softmax_scale=None,
                      k_scale_per_head=None, v_scale_per_head=None, q_len=1, lse=None,
                      page_indptr=None, tree_mask=None) -> L20PdFp8Args:
    """Fill ``l20_pd_fp8_args`` from tensors (same argument order as the fp8 op).

    The cache dtype picks ``kv_dtype`` (fp8 e4m3fn or e5m2, fp16 or bf16).  With
    ``page_indptr`` [B+1], ``block_table`` is the flat CSR page list.

    The struct holds raw device pointers; it also keeps a reference to every
    tensor it points into, so none of them is freed (and its memory handed to
    another tensor by the caching allocator) while the struct is alive."""
    a = L20PdFp8Args()
    a._tensors = tuple(t for t in (query, key_cache, value_cache, block_table, seq_lens, partial_output,
                                   partial_max, partial_sum, output, k_scale_per_head, v_scale_per_head, lse,
                                   page_indptr, tree_mask) if t is not None)
    a.kv_dtype = _kv_code(key_cache)
    a.query = query.data_ptr()
    a.query_dtype = _dtype_code(query)
    a.q_stride_row, a.q_stride_head = query.stride(0), query.stride(1)
    a.key_cache = key_cache.data_ptr()
    a.k_stride_page, a.k_stride_token, a.k_stride_head = key_cache.stride()[:3]
    a.value_cache = value_cache.data_ptr()
    a.v_stride_page, a.v_stride_token, a.v_stride_head = value_cache.stride()[:3]
    a.num_pages, a.page_size = key_cache.shape[0], key_cache.shape[1]
    a.block_table = block_table.data_ptr()
    if page_indptr is not None:
        a.page_indptr = page_indptr.data_ptr()
    else:
        a.bt_stride_row, a.bt_max_pages = block_table.stride(0), block_table.shape[1]
    a.seq_lens = seq_lens.data_ptr()
    if partial_output is not None:
        a.partial_output = partial_output.data_ptr()
        a.partial_dtype = _dtype_code(partial_output)
        a.po_stride_row, a.po_stride_head, a.po_stride_split = partial_output.stride()[:3]
        a.partial_splits = partial_output.shape[2]
        a.partial_max = partial_max.data_ptr()
        a.pm_stride_row, a.pm_stride_head, a.pm_stride_split = partial_max.stride()
        a.partial_sum = partial_sum.data_ptr()
        a.ps_stride_row, a.ps_stride_head, a.ps_stride_split = partial_sum.stride()
    a.output = output.data_ptr()
    a.o_stride_row, a.o_stride_head = output.stride(0), output.stride(1)
    if lse is not None:
        a.lse = lse.data_ptr()
        a.lse_stride_row, a.lse_stride_head = lse.stride()
    a.k_scale, a.v_scale = float(k_scale), float(v_scale)
    if k_scale_per_head is not None:
        a.k_scale_per_head = k_scale_per_head.data_ptr()
    if v_scale_per_head is not None:
        a.v_scale_per_head = v_scale_per_head.data_ptr()
    a.softmax_scale = 0.0 if softmax_scale is None else float(softmax_scale)
    a.batch = query.shape[0] // q_len
    a.q_len = q_len
    a.num_q_heads, a.head_dim = query.shape[1], query.shape[2]
    a.num_kv_heads = key_cache.shape[2]
    a.max_seq_len, a.split_size = int(max_seq_len), int(split_size)
    if tree_mask is not None:
        a.tree_mask = tree_mask.data_ptr()
        a.tree_mask_stride_batch = tree_mask.stride(0) if tree_mask.dim() == 2 else 0
    return a


def _call(name: str, args: L20PdFp8Args, stream: int, lib: Optional[ctypes.CDLL]) -> None:
    lib = lib or load()
    rc = getattr(lib, name)(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != L20_PD_OK:
        raise RuntimeError(last_error(lib))


def split_out(args: L20PdFp8Args, stream: int = 0, lib: Optional[ctypes.CDLL] = None) -> None:
    """Call ``l20_pd_fp8_e4m3_split_out`` (fp8 caches) or ``l20_pd_split_out`` (16-bit
    caches); raise RuntimeError with the library's message on failure."""
    fp8 = args.kv_dtype in (L20_PD_KV_FP8_E4M3, L20_PD_KV_FP8_E5M2)
    name = "l20_pd_fp8_e4m3_split_out" if fp8 else "l20_pd_split_out"
    _call(name, args, stream, lib)


def split_out_noalloc(args: L20PdFp8Args, stream: int = 0, lib: Optional[ctypes.CDLL] = None) -> None:
    """Call ``l20_pd_fp8_e4m3_split_out_noalloc``: the split partials go to the
    library's own per-device scratch (the struct's partial_* fields are ignored)."""
    _call("l20_pd_fp8_e4m3_split_out_noalloc", args, stream, lib)


def partial(args: L20PdFp8Args, stream: int = 0, lib: Optional[ctypes.CDLL] = None) -> None:
    """Enqueue only the split-KV partial kernel."""
    _call("l20_pd_fp8_e4m3_partial", args, stream, lib)


def merge(args: L20PdFp8Args, stream: int = 0, lib: Optional[ctypes.CDLL] = None) -> None:
    """Enqueue only the LSE merge kernel."""
    _call("l20_pd_fp8_e4m3_merge", args, stream, lib)


def device_errors(clear: bool = False, lib: Optional[ctypes.CDLL] = None) -> int:
    """``l20_pd_device_errors``: OR of the L20_PD_DEVERR_* codes the partial
    kernel recorded on the current device (synchronizes it)."""
    lib = lib or load()
    rc = lib.l20_pd_device_errors(1 if clear else 0)
    if rc < 0:
        raise RuntimeError(last_error(lib))
    return rc


def set_spin_limit(polls: int, lib: Optional[ctypes.CDLL] = None) -> None:
    """``l20_pd_set_spin_limit`` (0 restores the default)."""
    lib = lib or load()
    if lib.l20_pd_set_spin_limit(int(polls)) != L20_PD_OK:
        raise RuntimeError(last_error(lib))


def single_launch(args: L20PdFp8Args, lib: Optional[ctypes.CDLL] = None) -> bool:
    """``l20_pd_single_launch``: whether ``split_out(args)`` runs as the single
    launch on the current device (the workspace is then unused)."""
    lib = lib or load()
    rc = lib.l20_pd_single_launch(ctypes.byref(args))
    if rc < 0:
        raise RuntimeError(last_error(lib))
    return rc == 1


def launch_path(args: L20PdFp8Args, lib: Optional[ctypes.CDLL] = None) -> int:
    """``l20_pd_single_launch``'s code: 1 the single launch (no workspace, no
    merge), 2 the single-launch kernel's split mode for the partial stage
    (then the merge), 0 the persistent partial kernel and the merge."""
    lib = lib or load()
    rc = lib.l20_pd_single_launch(ctypes.byref(args))
    if rc < 0:
        raise RuntimeError(last_error(lib))
    return int(rc)


def set_queue_counters(value: int, lib: Optional[ctypes.CDLL] = None) -> None:
    """``l20_pd_set_queue_counters``: every work-queue counter of the current
    device set to ``value`` (a test hook; ``device_errors(clear=True)`` zeroes
    them)."""
    lib = lib or load()
    if lib.l20_pd_set_queue_counters(int(value)) != L20_PD_OK:
        raise RuntimeError(last_error(lib))


def check(args: L20PdFp8Args, lib: Optional[ctypes.CDLL] = None) -> None:
    lib = lib or load()
    if lib.l20_pd_fp8_e4m3_check(ctypes.byref(args)) != L20_PD_OK:
        raise RuntimeError(last_error(lib))


def tree_suffix_args_from_tensors(query, suffix_key, suffix_value, ancestor_mask, prefix_output, prefix_lse,
                                  output, softmax_scale: float) -> L20PdTreeSuffixArgs:
    """Fill ``l20_pd_tree_suffix_args``: query/prefix_output/output [B, S, Hq, D],
    suffix_key/value [B, S, Hkv, D], ancestor_mask bool [S, S], prefix_lse fp32
    [B, S, Hq].  Keeps references to the tensors on the struct."""
    a = L20PdTreeSuffixArgs()
    a._tensors = (query, suffix_key, suffix_value, ancestor_mask, prefix_output, prefix_lse, output)
    for name, t in (("query", query), ("suffix_key", suffix_key), ("suffix_value", suffix_value),
                    ("prefix_output", prefix_output), ("output", output)):
        if t.stride(-1) != 1:
            raise ValueError(f"{name}: head_dim must be the contiguous dimension")
    a.query = query.data_ptr()
    a.q_stride_batch, a.q_stride_draft, a.q_stride_head = query.stride()[:3]
    a.query_dtype = _dtype_code(query)
    a.suffix_key = suffix_key.data_ptr()
    a.sk_stride_batch, a.sk_stride_draft, a.sk_stride_head = suffix_key.stride()[:3]
    a.suffix_value = suffix_value.data_ptr()
    a.sv_stride_batch, a.sv_stride_draft, a.sv_stride_head = suffix_value.stride()[:3]
    a.ancestor_mask = ancestor_mask.data_ptr()
    a.mask_stride_row, a.mask_stride_col = ancestor_mask.stride()
    a.prefix_output = prefix_output.data_ptr()
    a.po_stride_batch, a.po_stride_draft, a.po_stride_head = prefix_output.stride()[:3]
    a.prefix_dtype = _dtype_code(prefix_output)
    a.prefix_lse = prefix_lse.data_ptr()
    a.pl_stride_batch, a.pl_stride_draft, a.pl_stride_head = prefix_lse.stride()
    a.output = output.data_ptr()
    a.o_stride_batch, a.o_stride_draft, a.o_stride_head = output.stride()[:3]
    a.softmax_scale = float(softmax_scale)
    a.batch, a.draft_length, a.num_q_heads, a.head_dim = query.shape
    a.num_kv_heads = suffix_key.shape[2]
    return a


def tree_suffix_merge(args: L20PdTreeSuffixArgs, stream: int = 0, lib: Optional[ctypes.CDLL] = None) -> None:
    """Call ``l20_pd_tree_suffix_merge``; raise RuntimeError with the library's message on failure."""
    lib = lib or load()
    if lib.l20_pd_tree_suffix_merge(ctypes.byref(args), ctypes.c_void_p(stream)) != L20_PD_OK:
        raise RuntimeError(last_error(lib))
