"""The C-ABI library loads on the CPU and exports every symbol the header declares.

No compute calls: this runs without a GPU.
"""
import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "vllm_apple_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vaa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from vllm_apple_amd import _lib

    if not _lib.library_path().exists():
        import vllm_apple_amd

        vllm_apple_amd.build_library(verbose=False)
    return _lib.load()


def test_header_declares_the_expected_entry_points():
    names = declared_functions()
    for must in ("vaa_write_kv_batch", "vaa_write_kv_single", "vaa_kv_write_slots",
                 "vaa_kv_write_decode", "vaa_paged_attention_decode",
                 "vaa_paged_attention_decode_workspace_size", "vaa_paged_attention_prefill",
                 "vaa_rmsnorm", "vaa_rope_neox", "vaa_silu_mul", "vaa_build_token_index",
                 "vaa_build_slot_mapping", "vaa_last_error", "vaa_abi_version"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_python_binding_covers_the_header(lib):
    from vllm_apple_amd import _lib

    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_params_struct_layout_matches_header(tmp_path):
    """The ctypes mirror of vaa_attn_params has the header's size and field
    offsets, as gcc lays the struct out from include/vllm_apple_amd.h."""
    import shutil
    import subprocess

    from vllm_apple_amd import _lib

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    names = [f[0] for f in _lib.VaaAttnParams._fields_]
    prog = tmp_path / "layout.c"
    prog.write_text(
        "#include <stdio.h>\n#include <stddef.h>\n#include \"vllm_apple_amd.h\"\n"
        "int main(void) {\n  printf(\"%zu\\n\", sizeof(vaa_attn_params));\n"
        + "".join(f'  printf("%zu\\n", offsetof(vaa_attn_params, {n}));\n' for n in names)
        + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{REPO / 'include'}", str(prog), "-o", str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(_lib.VaaAttnParams)
    assert got[1:] == [getattr(_lib.VaaAttnParams, n).offset for n in names]


def test_version_and_error_string_without_gpu(lib):
    assert lib.vaa_abi_version() == 5
    from vllm_apple_amd import _lib

    assert isinstance(_lib.last_error(), str)


def test_argument_errors_are_reported_without_touching_the_gpu(lib):
    """Bad arguments return VAA_ERR_INVALID_ARG / UNSUPPORTED before any launch."""
    from vllm_apple_amd import _lib

    p = _lib.VaaAttnParams()
    # Head sizes: any multiple of 8 up to 128.
    for bad in (100, 136, 0):
        p.head_size = bad
        st = lib.vaa_paged_attention_decode(ctypes.byref(p), None, None, None, None, None,
                                            None, None, None, None, 0, None)
        assert st == _lib.VAA_ERR_UNSUPPORTED
        assert f"head_size={bad}" in _lib.last_error()
        st = lib.vaa_paged_attention_prefill(ctypes.byref(p), None, None, None, None, None,
                                             None, None, 0, None)
        assert st == _lib.VAA_ERR_UNSUPPORTED and f"head_size={bad}" in _lib.last_error()
    p.head_size, p.block_size = 80, 16
    st = lib.vaa_paged_attention_decode(ctypes.byref(p), None, None, None, None, None, None,
                                        None, None, None, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG  # head size accepted; the zeroed heads are not
    assert "heads" in _lib.last_error()
    p.head_size, p.block_size = 100, 0
    st = lib.vaa_paged_attention_decode(ctypes.byref(p), None, None, None, None, None, None,
                                        None, None, None, 0, None)
    with pytest.raises(NotImplementedError):
        _lib.check(st, "decode")
    st = lib.vaa_rmsnorm(None, None, None, None, 4, 0, 0, 0, 0, 1e-5, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG
    with pytest.raises(ValueError):
        _lib.check(st, "rmsnorm")
    p.head_size = 128
    p.block_size = 0
    st = lib.vaa_paged_attention_decode(ctypes.byref(p), None, None, None, None, None, None,
                                        None, None, None, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG and "block_size=0" in _lib.last_error()
    # Any positive block size is accepted (rows of a tile find their own
    # blocks); the zeroed heads are what is refused next.
    p.block_size = 8
    st = lib.vaa_paged_attention_decode(ctypes.byref(p), None, None, None, None, None, None,
                                        None, None, None, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG and "heads" in _lib.last_error()


def test_zero_sized_calls_are_noops(lib):
    from vllm_apple_amd import _lib

    p = _lib.VaaAttnParams()
    p.num_kv_heads, p.head_size, p.block_size, p.num_blocks = 2, 64, 16, 4
    assert lib.vaa_kv_write_slots(ctypes.byref(p), None, None, None, 0, None, None, 0, None) == 0
    assert lib.vaa_silu_mul(None, None, None, 0, 0, None) == 0
    assert lib.vaa_build_token_index(None, None, 0, 0, None, None, None) == 0


def test_dtype_and_epilogue_argument_errors(lib):
    """dtype outside {F16, BF16} and bad epilogue shapes are refused before any launch."""
    from vllm_apple_amd import _lib

    p = _lib.VaaAttnParams()
    p.head_size, p.block_size, p.num_kv_heads, p.num_query_heads = 128, 16, 8, 32
    p.queries_per_kv, p.num_seqs, p.max_blocks_per_seq, p.num_blocks = 4, 1, 4, 4
    p.dtype = 7
    st = lib.vaa_paged_attention_decode(ctypes.byref(p), None, None, None, None, None, None,
                                        None, None, None, 0, None)
    assert st == _lib.VAA_ERR_UNSUPPORTED and "dtype=7" in _lib.last_error()
    st = lib.vaa_kv_write_slots(ctypes.byref(p), None, None, None, 0, None, None, 1, None)
    assert st == _lib.VAA_ERR_UNSUPPORTED
    p.dtype = _lib.VAA_DTYPE_BF16
    # rotary_dim not a multiple of 16
    st = lib.vaa_qkv_epilogue(ctypes.byref(p), None, None, None, None, None, None, 24, 16,
                              None, None, 0, None, None, 3, None)
    assert st == _lib.VAA_ERR_UNSUPPORTED and "rotary_dim=24" in _lib.last_error()
    # null tensors
    st = lib.vaa_qkv_epilogue(ctypes.byref(p), None, None, None, None, None, None, 128, 16,
                              None, None, 0, None, None, 3, None)
    assert st == _lib.VAA_ERR_INVALID_ARG and "null pointer" in _lib.last_error()
    # zero tokens is a no-op
    assert lib.vaa_qkv_epilogue(ctypes.byref(p), None, None, None, None, None, None, 128, 16,
                                None, None, 0, None, None, 0, None) == 0


def test_topk_argument_errors(lib):
    """k outside 1..256 or above vocab_size, short strides, odd pointers and a
    missing workspace are refused before any launch; zero tokens is a no-op."""
    from vllm_apple_amd import _lib

    fake = 0x10000  # never dereferenced: every call below fails its checks first
    ws = ctypes.c_size_t(0)

    def call(lg, T, V, rs, k, os_, w=None, wb=0):
        return lib.vaa_topk_logits(lg, T, V, rs, k, fake, fake, os_, w, wb, None)

    st = call(fake, 4, 1000, 1000, 257, 257)
    assert st == _lib.VAA_ERR_UNSUPPORTED and "k=257" in _lib.last_error()
    assert call(fake, 4, 10, 10, 11, 11) == _lib.VAA_ERR_UNSUPPORTED
    st = call(fake, 4, 1000, 999, 8, 8)
    assert st == _lib.VAA_ERR_INVALID_ARG and "row_stride" in _lib.last_error()
    assert call(fake, 4, 1000, 1000, 8, 7) == _lib.VAA_ERR_INVALID_ARG
    st = call(fake + 1, 4, 1000, 1000, 8, 8)
    assert st == _lib.VAA_ERR_INVALID_ARG and "2-byte aligned" in _lib.last_error()
    st = call(None, 4, 1000, 1000, 8, 8)
    assert st == _lib.VAA_ERR_INVALID_ARG and "null pointer" in _lib.last_error()
    assert call(None, 0, 1000, 1000, 8, 8) == 0
    # A vocabulary beyond what one merge holds for this k.
    st = lib.vaa_topk_workspace_size(4, 16384 * 16 + 1, 256, ctypes.byref(ws))
    assert st == _lib.VAA_ERR_UNSUPPORTED and "too large" in _lib.last_error()
    # A split row needs the workspace; a short one is refused.
    assert lib.vaa_topk_workspace_size(32, 128256, 50, ctypes.byref(ws)) == 0
    assert ws.value > 0 and ws.value % (32 * 50 * 8) == 0
    st = call(fake, 32, 128256, 128256, 50, 50)
    assert st == _lib.VAA_ERR_WORKSPACE and "workspace" in _lib.last_error()
    assert call(fake, 32, 128256, 128256, 50, 50, fake, ws.value - 8) == _lib.VAA_ERR_WORKSPACE


def test_topk_workspace_size(lib):
    """No workspace when a row is one chunk (<= 4096 columns) and the batch
    alone fills the GPU; otherwise T * S * k * 8 bytes, S chunks of <= 16384
    columns whose S * k survivors fit the merge (<= 4096)."""
    ws = ctypes.c_size_t(0)
    assert lib.vaa_topk_workspace_size(4096, 4096, 50, ctypes.byref(ws)) == 0
    assert ws.value == 0
    assert lib.vaa_topk_workspace_size(3, 8, 8, ctypes.byref(ws)) == 0 and ws.value == 0
    for T, V, k in ((32, 128256, 50), (256, 151936, 256), (1, 262144, 256), (9, 32000, 1)):
        assert lib.vaa_topk_workspace_size(T, V, k, ctypes.byref(ws)) == 0
        S = ws.value // (T * k * 8)
        assert ws.value == T * S * k * 8 and S >= 2
        assert S * k <= 4096 and -(-V // S) <= 16384


def test_add_rmsnorm_argument_errors(lib):
    """Output over the residual, short strides and null pointers are refused
    before any launch; zero tokens is a no-op."""
    from vllm_apple_amd import _lib

    a, b = 0x10000, 0x20000  # never dereferenced
    st = lib.vaa_add_rmsnorm(a, b, a, b, 4, 128, 128, 128, 128, 1e-6, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG and "alias" in _lib.last_error()
    st = lib.vaa_add_rmsnorm(a, b, a, a, 4, 128, 128, 64, 128, 1e-6, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG and "stride" in _lib.last_error()
    st = lib.vaa_add_rmsnorm(a, None, a, a, 4, 128, 128, 128, 128, 1e-6, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG and "null" in _lib.last_error()
    assert lib.vaa_add_rmsnorm(None, None, None, None, 0, 128, 128, 128, 128, 1e-6, 0, None) == 0


def test_layer_op_dtype_errors(lib):
    """A dtype outside {F16, BF16} is refused by every layer op before any launch."""
    from vllm_apple_amd import _lib

    a = 0x10000  # never dereferenced
    assert lib.vaa_rmsnorm(a, a, a, None, 4, 128, 128, 128, 0, 1e-6, 5,
                           None) == _lib.VAA_ERR_UNSUPPORTED
    assert "dtype=5" in _lib.last_error()
    assert lib.vaa_add_rmsnorm(a, a + 64, a, a, 4, 128, 128, 128, 128, 1e-6, 2,
                               None) == _lib.VAA_ERR_UNSUPPORTED
    assert lib.vaa_rope_neox(a, None, a, a, a, 4, 2, 0, 64, 64, 128, 0, 16, 9,
                             None) == _lib.VAA_ERR_UNSUPPORTED
    assert lib.vaa_silu_mul(a, a, a, 16, -1, None) == _lib.VAA_ERR_UNSUPPORTED
    assert lib.vaa_silu_mul_2d(a, a, a, 2, 16, 16, 16, 16, 3, None) == _lib.VAA_ERR_UNSUPPORTED


def test_balanced_shared_workspace(lib):
    """The shared balanced split plans two workgroups per CU: its workspace
    holds more partial rows than the one-per-CU split; other negative
    partition sizes are refused."""
    from vllm_apple_amd import _lib

    p = _lib.VaaAttnParams()
    p.head_size, p.block_size, p.num_kv_heads, p.num_query_heads = 128, 16, 8, 32
    p.queries_per_kv, p.num_seqs, p.max_blocks_per_seq, p.num_blocks = 4, 56, 1024, 8192
    p.max_seq_len = 16384
    part = ctypes.c_int32(0)
    p.partition_size = _lib.VAA_PARTITION_BALANCED
    one = lib.vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part))
    assert part.value == _lib.VAA_PARTITION_BALANCED
    p.partition_size = _lib.VAA_PARTITION_BALANCED_SHARED
    two = lib.vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part))
    assert part.value == _lib.VAA_PARTITION_BALANCED_SHARED
    assert two > one > 0
    p.partition_size = -3
    assert lib.vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part)) == 0
    # Fixed partitions index the grid's y dimension: at most 65535 of them.
    p.partition_size = 128
    p.max_blocks_per_seq = 1 << 20
    p.max_seq_len = 128 * 65535
    assert lib.vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part)) > 0
    p.max_seq_len = 128 * 65535 + 1
    assert lib.vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part)) == 0
    st = lib.vaa_paged_attention_decode(ctypes.byref(p), None, None, None, None, None, None,
                                        None, None, None, 0, None)
    assert st != 0


def test_prefill_split_arguments(lib):
    """The split prefill sizes its partials from max_seq_len, needs no
    workspace when max_seq_len fits one piece, and refuses split sizes that
    are not positive multiples of 64 before any launch."""
    from vllm_apple_amd import _lib

    p = _lib.VaaAttnParams()
    p.head_size, p.block_size, p.num_kv_heads, p.num_query_heads = 128, 16, 8, 32
    p.queries_per_kv, p.num_seqs, p.max_blocks_per_seq, p.num_blocks = 4, 8, 1024, 8192
    p.max_seq_len = 16384
    size = lib.vaa_paged_attention_prefill_workspace_size
    assert size(ctypes.byref(p), 2048, 4096) == 2048 * 32 * 4 * (128 + 2) * 4
    assert size(ctypes.byref(p), 2048, 16384) == 0  # one piece
    assert size(ctypes.byref(p), 2048, 100) == 0 and "multiple of 64" in _lib.last_error()
    st = lib.vaa_paged_attention_prefill_split(ctypes.byref(p), None, None, None, None, None,
                                               None, None, 16, 96, None, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG and "split_keys=96" in _lib.last_error()
    st = lib.vaa_paged_attention_prefill_split(ctypes.byref(p), None, None, None, None, None,
                                               None, None, 16, 0, None, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG
    p.max_blocks_per_seq = 1 << 20
    p.max_seq_len = 64 * 1025  # more than 1024 pieces of 64 keys
    st = lib.vaa_paged_attention_prefill_split(ctypes.byref(p), None, None, None, None, None,
                                               None, None, 16, 64, None, 0, None)
    assert st == _lib.VAA_ERR_UNSUPPORTED


def test_wide_groups_and_merge_arguments(lib):
    """GQA groups above 16 heads have a workspace size (head chunks), the
    state merge checks its arguments, and the single-token KV write rejects an
    offset or block outside the pool before any launch."""
    from vllm_apple_amd import _lib

    p = _lib.VaaAttnParams()
    p.head_size, p.block_size, p.num_kv_heads, p.num_query_heads = 128, 16, 1, 48
    p.queries_per_kv, p.num_seqs, p.max_blocks_per_seq, p.num_blocks = 48, 4, 64, 256
    p.max_seq_len = 1024
    part = ctypes.c_int32(0)
    p.partition_size = 128
    n = lib.vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part))
    assert n == 4 * 48 * 8 * 130 * 4 and part.value == 128
    p.partition_size = -1
    n = lib.vaa_paged_attention_decode_workspace_size(ctypes.byref(p), ctypes.byref(part))
    assert n > 0
    st = lib.vaa_merge_attn_states(None, None, None, 2, 0, 4, 128, None, 0, 0, None, 0, None)
    assert st == _lib.VAA_ERR_INVALID_ARG
    st = lib.vaa_merge_attn_states(None, None, None, 2, 4, 4, 128, None, 0, 0, None, 9, None)
    assert st == _lib.VAA_ERR_UNSUPPORTED
    assert lib.vaa_merge_attn_states(None, None, None, 0, 4, 4, 128, None, 0, 0, None, 0,
                                     None) == 0
    # num_seqs is the grid's y dimension (at most 65535); num_heads (x) may be large.
    buf0 = ctypes.create_string_buffer(16)
    a0 = ctypes.addressof(buf0)
    st = lib.vaa_merge_attn_states(a0, a0, None, 65536, 4, 4, 128, a0, 0, 0, None, 0, None)
    assert st == _lib.VAA_ERR_UNSUPPORTED and "num_seqs=65536" in _lib.last_error()
    buf = ctypes.create_string_buffer(64)
    a = ctypes.addressof(buf)
    # kernel layout, KV 2, bs 16, D 64: offsets 0..15 are inside a block.
    sb, sh, st_ = 2 * 16 * 64, 16 * 64, 64
    for b, o in ((3, 16), (3, -1), (-1, 0), (8, 0)):
        st = lib.vaa_write_kv_single(a, a, a, a, b, o, 2, 64, sb, sh, st_, 8, None)
        assert st == _lib.VAA_ERR_INVALID_ARG, (b, o)
        assert "vaa_write_kv_single" in _lib.last_error()
