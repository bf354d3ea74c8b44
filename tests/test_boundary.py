"""The drop-in boundary on CPU: C ABI exports and validation, the torch op
schema and fake implementation, and the hook-facing Python API's contract.
No kernel is launched here.
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import l20_pd_cabi as cabi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "l20_paged_decode.h"
HIP_SRC = ROOT / "single-gpu-inference-lab_amd" / "csrc" / "l20_paged_decode_fp8.hip"
OPS_SRC = ROOT / "single-gpu-inference-lab_amd" / "csrc" / "l20_paged_decode_ops.cpp"

REFERENCE_SCHEMA_PREFIX = (
    "l20_stack::paged_decode_fp8_e4m3_split_out(Tensor query, Tensor key_cache, Tensor value_cache, "
    "Tensor block_table, Tensor seq_lens, Tensor(a!) partial_output, Tensor(b!) partial_max, "
    "Tensor(c!) partial_sum, Tensor(d!) output, float k_scale, float v_scale, int max_seq_len, "
    "int split_size"
)


def header_functions():
    """Every function declared in include/*.h."""
    names = set()
    for header in sorted(HEADER.parent.glob("*.h")):
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(l20_pd_\w+)\s*\(", header.read_text(), re.M))
    return sorted(names)


def test_library_exports_every_header_symbol():
    lib = cabi.load()
    declared = header_functions()
    assert declared, "no declarations parsed from the header"
    assert sorted(cabi.EXPORTED) == declared
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.l20_pd_abi_version() == cabi.ABI_VERSION == 4


def test_num_splits_and_default_split_size():
    lib = cabi.load()
    assert lib.l20_pd_num_splits(257, 128) == 3
    assert lib.l20_pd_num_splits(256, 128) == 2
    assert lib.l20_pd_num_splits(0, 128) == 0
    for b, h, s in [(128, 4, 8192), (2, 8, 131072), (4, 2, 512), (1, 1, 16)]:
        split = lib.l20_pd_default_split_size(b, h, s, 256)
        assert 64 <= split <= 1024 and split % 16 == 0
    # long contexts take the largest split; serving batches the hook's 512;
    # short contexts keep ~8 splits per sequence, and halve the split while the
    # items fill at most half the grid (32 x 8 items on 1024 slots -> 128)
    assert lib.l20_pd_default_split_size(2, 8, 131072, 256) == 1024
    assert lib.l20_pd_default_split_size(128, 4, 8192, 256) == 512
    assert lib.l20_pd_default_split_size(64, 2, 2048, 256) == 1024  # 512 triples at 512, 256 at 1024
    assert lib.l20_pd_default_split_size(64, 2, 2048, 512) == 512  # 512 triples on 512 CUs
    assert lib.l20_pd_default_split_size(128, 2, 2048, 256) == 256  # 512 triples at 1024: the persistent rules
    # the first of 256, 512 and 1024 whose (split, sequence, KV head) triples
    # of a batch beyond 1024 tokens fit the CUs (and at 512 / 1024 tokens fill
    # at least / more than half of them: the single-launch kernel's split
    # mode): 32 x 2 x 4 = 256 triples at 512
    assert lib.l20_pd_default_split_size(32, 2, 2048, 256) == 512
    assert lib.l20_pd_default_split_size(1, 8, 16384, 256) == 512
    assert lib.l20_pd_default_split_size(16, 2, 8192, 256) == 1024  # 512 triples at 512, 256 at 1024
    assert lib.l20_pd_default_split_size(16, 2, 2048, 256) == 256  # 256 triples at 256
    assert lib.l20_pd_default_split_size(8, 2, 2048, 256) == 256  # 128 triples at 256
    assert lib.l20_pd_default_split_size(1, 2, 1100, 256) == 256  # 10 triples at 256: any count
    assert lib.l20_pd_default_split_size(16, 2, 4096, 256) == 512  # 512 triples at 256, 128 at 512
    assert lib.l20_pd_default_split_size(32, 2, 2048, 512) != 512  # 256 triples: half of 512 CUs
    assert lib.l20_pd_default_split_size(32, 2, 2048, 128) != 512  # 256 triples on 128 CUs
    assert lib.l20_pd_default_split_size(4, 2, 512, 256) == 64
    # doubled when that fits every item in one round of the persistent grid
    # (64 sequences x 4 splits on 256 one-workgroup CUs), never past 1024
    assert lib.l20_pd_default_split_size(64, 8, 4096, 256) == 1024
    assert lib.l20_pd_default_split_size(64, 8, 4096, 128) == 512
    assert lib.l20_pd_default_split_size(8, 8, 32768, 256) == 1024


def valid_args():
    """A well-formed argument block with fake (never dereferenced) pointers."""
    a = cabi.L20PdFp8Args()
    fake = 0x10000
    a.query, a.query_dtype, a.q_stride_row, a.q_stride_head = fake, cabi.L20_PD_BF16, 28 * 128, 128
    a.key_cache, a.k_stride_page, a.k_stride_token, a.k_stride_head = fake, 16 * 4 * 128, 4 * 128, 128
    a.value_cache, a.v_stride_page, a.v_stride_token, a.v_stride_head = fake, 16 * 4 * 128, 4 * 128, 128
    a.num_pages, a.page_size = 1000, 16
    a.block_table, a.bt_stride_row, a.bt_max_pages = fake, 64, 64
    a.seq_lens = fake
    a.partial_output, a.partial_dtype = fake, cabi.L20_PD_FP32
    a.po_stride_row, a.po_stride_head, a.po_stride_split, a.partial_splits = 28 * 4 * 128, 4 * 128, 128, 4
    a.partial_max, a.pm_stride_row, a.pm_stride_head, a.pm_stride_split = fake, 28 * 4, 4, 1
    a.partial_sum, a.ps_stride_row, a.ps_stride_head, a.ps_stride_split = fake, 28 * 4, 4, 1
    a.output, a.o_stride_row, a.o_stride_head = fake, 28 * 128, 128
    a.k_scale = a.v_scale = 0.01
    a.batch, a.q_len, a.num_q_heads, a.num_kv_heads, a.head_dim = 8, 1, 28, 4, 128
    a.max_seq_len, a.split_size = 1024, 256
    return a


def test_check_accepts_valid_arguments():
    cabi.check(valid_args())


def test_args_from_tensors_keeps_its_tensors_alive():
    """The struct holds raw pointers: the tensors behind them must outlive any
    temporaries of the caller (a freed workspace would be handed to the next
    allocation while the struct still points into it)."""
    import gc
    import weakref

    import torch

    q = torch.zeros(4, 8, 128, dtype=torch.bfloat16)
    kc = torch.zeros(10, 16, 2, 128, dtype=torch.uint8).view(torch.float8_e4m3fn)
    bt = torch.zeros(4, 4, dtype=torch.int32)
    lens = torch.full((4,), 40, dtype=torch.int32)

    def build():
        po = torch.empty(4, 8, 2, 128)
        pm, ps, out = torch.empty(4, 8, 2), torch.empty(4, 8, 2), torch.empty_like(q)
        lse = torch.empty(4, 8)
        refs = [weakref.ref(t) for t in (po, pm, ps, out, lse)]
        return cabi.args_from_tensors(q, kc, kc, bt, lens, po, pm, ps, out, 1.0, 1.0, 64, 64, lse=lse), refs

    a, refs = build()
    gc.collect()
    assert all(r() is not None for r in refs)
    assert a.partial_output == refs[0]().data_ptr() and a.lse == refs[4]().data_ptr()
    cabi.check(a)
    del a
    gc.collect()
    assert all(r() is None for r in refs)


BAD = [
    ("split_size", 48, "split_size must be a multiple of 16 from 64 through 1024"),
    ("split_size", 1040, "split_size must be a multiple of 16 from 64 through 1024"),
    ("split_size", 72, "split_size must be a multiple of 16 from 64 through 1024"),
    ("num_q_heads", 30, "Q heads must be divisible by KV heads"),
    ("partial_splits", 3, "partial output workspace has wrong shape"),
    ("partial_output", 0, "partial output workspace has wrong shape"),
    ("head_dim", 96, "NHD cache only"),
    ("page_size", 24, "page_size must be a multiple of 16 from 16 through 4096"),
    ("page_size", 8, "page_size must be a multiple of 16 from 16 through 4096"),
    ("page_size", 4112, "page_size must be a multiple of 16 from 16 through 4096"),
    # 32-token pages whose page stride is that of 16-token pages: not contiguous
    ("page_size", 32, "pages of more than 16 tokens must hold them contiguously"),
    ("query_dtype", cabi.L20_PD_FP32, "query must be bf16 or fp16"),
    ("q_len", 0, "q_len must be >= 1"),
    ("q_len", 5, "GQA group x q_len must be at most 32"),
    ("k_stride_token", 4 * 128 + 8, "K cache pointer and strides must be 16-byte aligned"),
    ("v_stride_head", 130, "V cache pointer and strides must be aligned"),
    ("q_stride_head", 132, "query pointer and strides must be 16-byte aligned"),
    ("bt_max_pages", 63, "block table has fewer pages than max_seq_len needs"),
    ("query", 0, "null tensor pointer"),
    ("num_pages", 0, "K/V cache has no pages"),
]


@pytest.mark.parametrize("field,value,message", BAD)
def test_check_rejects_bad_arguments(field, value, message):
    a = valid_args()
    setattr(a, field, value)
    with pytest.raises(RuntimeError, match=re.escape(message)):
        cabi.check(a)
    # the launching entry point validates identically and enqueues nothing
    lib = cabi.load()
    assert lib.l20_pd_fp8_e4m3_split_out(ctypes.byref(a), None) == cabi.L20_PD_EINVAL
    assert message in cabi.last_error(lib)


def test_check_accepts_pages_of_a_multiple_of_16_tokens():
    # 64-token pages, contiguous: the block table then needs a quarter of the entries
    a = valid_args()
    a.page_size = 64
    a.k_stride_page = a.v_stride_page = 64 * 4 * 128
    a.bt_max_pages = 16
    cabi.check(a)
    a.bt_max_pages = 15  # 960 tokens < max_seq_len 1024
    with pytest.raises(RuntimeError, match="block table has fewer pages than max_seq_len needs"):
        cabi.check(a)


def test_check_rejects_pair_count_beyond_int32():
    # the merge kernels index (query row, q head) pairs in 32 bits
    a = valid_args()
    a.num_q_heads = a.num_kv_heads = 1 << 30
    message = "batch x q_len x Q heads must be below 2^31"
    with pytest.raises(RuntimeError, match=re.escape(message)):
        cabi.check(a)
    lib = cabi.load()
    assert lib.l20_pd_fp8_e4m3_split_out(ctypes.byref(a), None) == cabi.L20_PD_EINVAL


def test_single_split_needs_no_workspace():
    a = valid_args()
    a.max_seq_len, a.split_size = 200, 256
    a.partial_output = a.partial_max = a.partial_sum = 0
    cabi.check(a)


def test_single_launch_rule(monkeypatch):
    """l20_pd_single_launch reports the path split_out takes, on the host (no
    GPU here: the CU count defaults to 256).  One launch for fp8 caches, one
    query tile, at most one (sequence, KV head) pair per CU and at most 1024
    tokens within reach, one or two query tiles; L20_PD_FUSED=0/1 overrides only
    the size rule."""
    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    assert cabi.single_launch(valid_args())  # 8 x 4 pairs, 1024 tokens
    longer = valid_args()
    longer.max_seq_len, longer.partial_splits, longer.bt_max_pages = 1040, 5, 80  # 1280 tokens within reach
    assert not cabi.single_launch(longer)
    many = valid_args()
    many.batch = 65  # 260 pairs
    assert not cabi.single_launch(many)
    drafts = valid_args()
    drafts.q_len = 4  # 7 x 4 = 28 query columns: two tiles (the checks allow at most 32)
    assert cabi.single_launch(drafts)
    half = valid_args()  # 16-bit caches: up to 640 tokens within reach
    half.kv_dtype, half.query_dtype = cabi.L20_PD_KV_FP16, cabi.L20_PD_FP16
    half.max_seq_len, half.split_size, half.partial_splits = 640, 128, 6
    half.po_stride_row, half.po_stride_head = 28 * 6 * 128, 6 * 128
    half.pm_stride_row = half.ps_stride_row = 28 * 6
    half.pm_stride_head = half.ps_stride_head = 6
    assert cabi.single_launch(half)
    half.max_seq_len = 656
    assert not cabi.single_launch(half)
    monkeypatch.setenv("L20_PD_FUSED", "1")
    assert cabi.single_launch(longer) and cabi.single_launch(many) and cabi.single_launch(drafts)
    monkeypatch.setenv("L20_PD_FUSED", "0")
    assert not cabi.single_launch(valid_args())
    bad = valid_args()
    bad.head_dim = 96
    with pytest.raises(RuntimeError):
        cabi.single_launch(bad)


def _with_split(a, split):
    """``a`` with its workspace shaped for ``split``: one slot per split."""
    n = -(-a.max_seq_len // split)
    a.split_size, a.partial_splits = split, n
    a.po_stride_row, a.po_stride_head, a.po_stride_split = 28 * n * 128, n * 128, 128
    a.pm_stride_row = a.ps_stride_row = 28 * n
    a.pm_stride_head = a.ps_stride_head = n
    return a


def test_split_mode_rule(monkeypatch):
    """l20_pd_single_launch returns 2 when the partial stage runs as the
    single-launch kernel's split mode (one workgroup per (split, sequence, KV
    head), merge after): 256-, 512- or 1024-token splits whose triples do not
    exceed the CUs (256 here, no GPU) and, at 512 (1024) tokens, fill at least
    (more than) half of them; L20_PD_FUSED_SPLIT=0/1 overrides the size rule,
    not the shape conditions."""
    monkeypatch.delenv("L20_PD_FUSED", raising=False)
    monkeypatch.delenv("L20_PD_FUSED_SPLIT", raising=False)
    a = valid_args()  # 28 query / 4 KV heads
    a.max_seq_len, a.bt_stride_row, a.bt_max_pages = 2048, 128, 128
    a.batch = 16
    _with_split(a, 512)
    assert cabi.launch_path(a) == 2  # 16 x 4 x 4 = 256 triples
    assert not cabi.single_launch(a)
    a.batch = 8  # 128 triples: half the CUs (enough at 256 and 512 tokens)
    assert cabi.launch_path(a) == 2
    a.batch = 7  # 112 triples
    assert cabi.launch_path(a) == 0
    a.batch = 17  # 272 triples
    assert cabi.launch_path(a) == 0
    a.batch = 16
    _with_split(a, 1024)  # 16 x 4 x 2 = 128 triples: at 1024 tokens, more than half are needed
    assert cabi.launch_path(a) == 0
    a.batch = 8
    a.max_seq_len, a.bt_stride_row, a.bt_max_pages = 8192, 512, 512
    _with_split(a, 1024)  # 8 x 4 x 8 = 256 triples
    assert cabi.launch_path(a) == 2
    a.max_seq_len, a.bt_stride_row, a.bt_max_pages = 2048, 128, 128
    a.batch = 16
    _with_split(a, 256)  # 16 x 4 x 8 = 512 triples: two rounds
    assert cabi.launch_path(a) == 0
    a.batch = 8
    assert cabi.launch_path(a) == 2  # 256 triples at 256-token splits (one block per wave)
    a.batch = 1
    assert cabi.launch_path(a) == 2  # 32 triples: any count at 256 tokens
    a.batch = 16
    assert cabi.launch_path(a) == 0
    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "1")
    assert cabi.launch_path(a) == 2
    _with_split(a, 384)  # 48 tokens per wave: not whole fp8 blocks
    assert cabi.launch_path(a) == 0
    monkeypatch.setenv("L20_PD_FUSED_SPLIT", "0")
    _with_split(a, 512)
    assert cabi.launch_path(a) == 0
    a.max_seq_len, a.bt_max_pages = 1024, 64  # within the single launch's reach
    monkeypatch.delenv("L20_PD_FUSED_SPLIT")
    _with_split(a, 512)
    a.batch = 32  # 128 pairs: the single launch first
    assert cabi.launch_path(a) == 1


def test_empty_batch_is_a_noop():
    a = valid_args()
    a.batch = 0
    lib = cabi.load()
    assert lib.l20_pd_fp8_e4m3_split_out(ctypes.byref(a), None) == cabi.L20_PD_OK


# ------------------------------------------------------------------ torch op
def test_torch_op_keeps_reference_schema_and_extends_it():
    import l20_paged_decode  # noqa: F401

    schema = str(torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out.default._schema)
    assert schema.startswith(REFERENCE_SCHEMA_PREFIX)
    for extra in ("float? softmax_scale=None", "Tensor? k_scale_per_head=None", "Tensor? v_scale_per_head=None",
                  "int q_len=1", "Tensor(e!)? lse=None"):
        assert extra in schema
    assert schema.endswith("-> Tensor(d!)")


def _meta_inputs(rows=4, hq=8, hkv=2, d=128, pages=32, splits=3):
    m = dict(device="meta")
    return (
        torch.empty(rows, hq, d, dtype=torch.bfloat16, **m),
        torch.empty(pages, 16, hkv, d, dtype=torch.float8_e4m3fn, **m),
        torch.empty(pages, 16, hkv, d, dtype=torch.float8_e4m3fn, **m),
        torch.empty(rows, 8, dtype=torch.int32, **m),
        torch.empty(rows, dtype=torch.int32, **m),
        torch.empty(rows, hq, splits, d, dtype=torch.float32, **m),
        torch.empty(rows, hq, splits, dtype=torch.float32, **m),
        torch.empty(rows, hq, splits, dtype=torch.float32, **m),
        torch.empty(rows, hq, d, dtype=torch.bfloat16, **m),
    )


def test_fake_impl_returns_output_alias_on_meta_tensors():
    import l20_paged_decode

    args = _meta_inputs()
    out = l20_paged_decode.paged_decode_fp8_e4m3_split_out(*args, 0.1, 0.1, 128, 64)
    assert out.shape == args[-1].shape and out.dtype == torch.bfloat16 and out.device.type == "meta"
    # legacy 13-positional-argument call through the dispatcher
    out2 = torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(*args, 0.1, 0.1, 128, 64)
    assert out2.shape == args[-1].shape


def test_fake_impl_traces_under_fake_tensor_mode():
    import l20_paged_decode
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode() as mode:
        args = [mode.from_tensor(torch.empty(t.shape, dtype=t.dtype)) for t in _meta_inputs()]
        out = l20_paged_decode.paged_decode_fp8_e4m3_split_out(*args, 0.1, 0.1, 128, 64, q_len=2)
        assert out.shape == args[-1].shape


def test_allocating_entry_points_of_the_reference_extension():
    """The reference's extension module (l20_paged_decode.cpp:145-156) exports
    paged_decode and paged_decode_split beside the three _out functions: this
    module has all five names, and the allocating two return a new output of
    the query's shape and dtype (here through the fake implementation, on meta
    tensors, with the split size taken from the block table's bound)."""
    import l20_paged_decode as ext

    for name in ("paged_decode", "paged_decode_split", "paged_decode_split_out", "paged_decode_split_indices_out",
                 "paged_decode_fp8_e4m3_split_out"):
        assert callable(getattr(ext, name)), name
    q = torch.empty(4, 16, 128, dtype=torch.float16, device="meta")
    kc = torch.empty(64, 16, 8, 128, dtype=torch.float16, device="meta")
    bt = torch.empty(4, 16, dtype=torch.int32, device="meta")
    sl = torch.empty(4, dtype=torch.int32, device="meta")
    for out in (ext.paged_decode(q, kc, kc, bt, sl), ext.paged_decode_split(q, kc, kc, bt, sl, 256, 64)):
        assert out.shape == q.shape and out.dtype == q.dtype and out.device.type == "meta"
    with pytest.raises(RuntimeError, match="invalid query"):
        ext.paged_decode_split(q[0], kc, kc, bt, sl, 256, 64)


def test_op_rejects_cpu_query_with_reference_message():
    import l20_paged_decode  # noqa: F401

    args = [torch.empty(t.shape, dtype=t.dtype) for t in _meta_inputs()]
    with pytest.raises((RuntimeError, NotImplementedError)):
        torch.ops.l20_stack.paged_decode_fp8_e4m3_split_out(*args, 0.1, 0.1, 128, 64)


# ------------------------------------------------------------------ hook API
def test_hook_api_requires_mi355x_and_fp8_cache():
    import l20_paged_split_kv as sk

    q = torch.empty(2, 8, 128, dtype=torch.bfloat16)
    kv = torch.empty(4, 16, 2, 128, dtype=torch.float8_e4m3fn)
    with pytest.raises(RuntimeError, match="requires an MI355X"):
        sk.l20_paged_split_kv_attention_fp8(q, kv, kv, torch.zeros(2, 4, dtype=torch.int32),
                                            torch.ones(2, dtype=torch.int32), k_scale=1.0, v_scale=1.0)
    assert sk.should_use_l20_paged_fp8_split_kv(8, 4096) is False  # closed, as in the reference


def test_workspace_allocation_shapes():
    import l20_paged_split_kv as sk

    q = torch.empty(12, 28, 128, dtype=torch.bfloat16)
    po, pm, ps, out = sk.allocate_l20_paged_split_kv_workspace(q, 1000, split_size=256)
    assert po.shape == (12, 28, 4, 128) and po.dtype == torch.float32
    assert pm.shape == ps.shape == (12, 28, 4)
    assert out.shape == q.shape and out.dtype == q.dtype


# ------------------------------------------------------------------ source contracts
def test_kernel_source_contracts():
    """The reference's source-string contract (tests/test_cuda_paged_decode_source.py:4-37),
    restated for this build's kernel and binding names."""
    src = HIP_SRC.read_text()
    ops = OPS_SRC.read_text()
    for name in ("pd_fp8_partial", "pd_merge", "split_size must be a multiple of 16 from 64 through 1024",
                 "Q heads must be divisible by KV heads", "partial output workspace has wrong shape",
                 "v_mfma", "__builtin_amdgcn_mfma_f32_16x16x32_bf16"):
        assert name in src, name
    for needle in ("TORCH_LIBRARY(l20_stack", "TORCH_LIBRARY_IMPL(l20_stack, CUDA", "query must be CUDA",
                   "K/V cache must be torch.float8_e4m3fn", "int32 block table", "int32 sequence lengths"):
        assert needle in ops, needle
    assert "hipMalloc" not in src and "hipMemset" not in src  # the op allocates nothing


# ------------------------------------------------------------------ fp16/bf16-KV siblings, CSR
# integrations/vllm/cuda/l20_paged_decode.cpp:121-127 (reference schema, kept verbatim)
REFERENCE_FP16_SCHEMA_PREFIX = (
    "l20_stack::paged_decode_split_out(Tensor query, Tensor key_cache, Tensor value_cache, "
    "Tensor block_table, Tensor seq_lens, Tensor(a!) partial_output, Tensor(b!) partial_max, "
    "Tensor(c!) partial_sum, Tensor(d!) output, int max_seq_len, int split_size"
)


def test_sibling_ops_keep_reference_schema_and_extend_it():
    import l20_paged_decode  # noqa: F401

    schema = str(torch.ops.l20_stack.paged_decode_split_out.default._schema)
    assert schema.startswith(REFERENCE_FP16_SCHEMA_PREFIX)
    for extra in ("float? softmax_scale=None", "int q_len=1", "Tensor(e!)? lse=None"):
        assert extra in schema
    csr = str(torch.ops.l20_stack.paged_decode_split_indices_out.default._schema)
    # argument order of l20_paged_decode_split_indices_out_cuda (l20_paged_decode.cu:600-612)
    assert csr.startswith(
        "l20_stack::paged_decode_split_indices_out(Tensor query, Tensor key_cache, Tensor value_cache, "
        "Tensor page_indptr, Tensor page_indices, Tensor seq_lens, Tensor(a!) partial_output, "
        "Tensor(b!) partial_max, Tensor(c!) partial_sum, Tensor(d!) output, int max_seq_len, int split_size")


def test_sibling_fakes_return_output_alias():
    import l20_paged_decode

    q, kc, vc, bt, sl, po, pm, ps, out = _meta_inputs()
    kc16 = torch.empty(kc.shape, dtype=torch.bfloat16, device="meta")
    r = l20_paged_decode.paged_decode_split_out(q, kc16, kc16, bt, sl, po, pm, ps, out, 128, 64)
    assert r.shape == out.shape and r.device.type == "meta"
    ip = torch.empty(q.shape[0] + 1, dtype=torch.int32, device="meta")
    idx = torch.empty(64, dtype=torch.int32, device="meta")
    r = l20_paged_decode.paged_decode_split_indices_out(q, kc16, kc16, ip, idx, sl, po, pm, ps, out, 128, 64)
    assert r.shape == out.shape


def test_check_16bit_caches_and_csr():
    lib = cabi.load()
    a = valid_args()
    a.kv_dtype = cabi.L20_PD_KV_BF16  # bf16 query, strides now in elements
    cabi.check(a)
    a.query_dtype = cabi.L20_PD_FP16
    with pytest.raises(RuntimeError, match="query and 16-bit K/V cache must have the same dtype"):
        cabi.check(a)
    a = valid_args()
    a.kv_dtype = 7
    with pytest.raises(RuntimeError, match="unknown K/V cache dtype"):
        cabi.check(a)
    # entry points accept only their cache types
    a = valid_args()
    assert lib.l20_pd_split_out(ctypes.byref(a), None) == cabi.L20_PD_EINVAL
    assert "fp16 or bf16" in cabi.last_error(lib)
    a.kv_dtype = cabi.L20_PD_KV_BF16
    assert lib.l20_pd_fp8_e4m3_split_out(ctypes.byref(a), None) == cabi.L20_PD_EINVAL
    assert "float8_e4m3fn" in cabi.last_error(lib)
    # a CSR page list needs no block-table row length
    a = valid_args()
    a.page_indptr, a.bt_max_pages = 0x10000, 0
    cabi.check(a)
    # 16-bit V rows need head_dim/16-element alignment (8 elements = 16 B at D=128)
    a = valid_args()
    a.kv_dtype = cabi.L20_PD_KV_BF16
    a.v_stride_head = 132
    with pytest.raises(RuntimeError, match="V cache pointer and strides must be aligned"):
        cabi.check(a)


def test_tree_suffix_check_validates_without_a_gpu():
    """l20_pd_tree_suffix_check (include/l20_tree_verify.h): the reference's limits
    (draft_length 1..64, integral GQA ratio) plus head_dim 64/128 and the dtypes."""
    lib = cabi.load()

    def args(**kw):
        a = cabi.L20PdTreeSuffixArgs()
        for name in ("query", "suffix_key", "suffix_value", "ancestor_mask", "prefix_output", "prefix_lse", "output"):
            setattr(a, name, 4096)  # never dereferenced by the check
        a.query_dtype = a.prefix_dtype = cabi.L20_PD_BF16
        a.softmax_scale = 0.125
        a.batch, a.draft_length, a.num_q_heads, a.num_kv_heads, a.head_dim = 2, 8, 28, 4, 128
        for k, v in kw.items():
            setattr(a, k, v)
        return ctypes.byref(a)

    assert lib.l20_pd_tree_suffix_check(args()) == cabi.L20_PD_OK
    assert lib.l20_pd_tree_suffix_check(args(prefix_dtype=cabi.L20_PD_FP32, head_dim=64)) == cabi.L20_PD_OK
    for kw, msg in [(dict(draft_length=65), "draft_length"), (dict(draft_length=0), "draft_length"),
                    (dict(head_dim=96), "head_dim"), (dict(num_kv_heads=3), "GQA"),
                    (dict(query_dtype=cabi.L20_PD_FP32), "bf16 or fp16"),
                    (dict(prefix_dtype=cabi.L20_PD_FP16), "prefix output"),
                    (dict(output=0), "null"), (dict(softmax_scale=0.0), "softmax_scale")]:
        assert lib.l20_pd_tree_suffix_check(args(**kw)) == cabi.L20_PD_EINVAL, kw
        assert msg in cabi.last_error(lib), (kw, cabi.last_error(lib))


def test_tree_suffix_merge_op_schema_and_fake():
    import l20_paged_decode  # noqa: F401

    schema = str(torch.ops.l20_stack.tree_suffix_merge.default._schema)
    assert "Tensor(a!) output" in schema and schema.endswith("-> ()")
    m = dict(device="meta")
    q = torch.empty(2, 4, 8, 128, dtype=torch.bfloat16, **m)
    kv = torch.empty(2, 4, 2, 128, dtype=torch.bfloat16, **m)
    mask = torch.empty(4, 4, dtype=torch.bool, **m)
    lse = torch.empty(2, 4, 8, dtype=torch.float32, **m)
    assert torch.ops.l20_stack.tree_suffix_merge(q, kv, kv, mask, q, lse, torch.empty_like(q), 0.1) is None
