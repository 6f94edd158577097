"""The C-ABI library loads without a GPU, exports every function that
include/parakeet_paged.h declares, and the ctypes structures match the header's
field order.  No kernel is launched here."""

import ctypes
import re
from pathlib import Path

import pytest

from parakeet_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "parakeet_paged.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(pk_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def _struct_fields(name):
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    m = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S)
    assert m, name
    fields = []
    for line in m.group(1).split(";"):
        line = line.strip()
        if not line:
            continue
        fields.append(line.split()[-1].lstrip("*"))
    return fields


def test_library_loads_and_versions():
    lib = _lib.lib()
    assert lib.pk_abi_version() == _lib.ABI_VERSION
    assert _lib.last_error() == ""


def test_every_declared_symbol_is_exported_and_bound():
    declared = _declared_functions()
    assert len(declared) >= 15, declared
    lib = _lib.lib()
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(_lib.SIGNATURES) == declared


@pytest.mark.parametrize(
    "cname,pyclass",
    [
        ("pk_paged_layout", _lib.PagedLayout),
        ("pk_kv_append_args", _lib.KvAppendArgs),
        ("pk_kv_gather_args", _lib.KvGatherArgs),
        ("pk_attn_args", _lib.AttnArgs),
        ("pk_mask_args", _lib.MaskArgs),
        ("pk_conv_args", _lib.ConvArgs),
        ("pk_resnorm_args", _lib.ResNormArgs),
        ("pk_fe_stream", _lib.FeStream),
        ("pk_fe_args", _lib.FeArgs),
        ("pk_sub_stream", _lib.SubStream),
        ("pk_sub_args", _lib.SubArgs),
        ("pk_rnnt_args", _lib.RnntArgs),
    ],
)
def test_struct_layout_matches_header(cname, pyclass):
    assert [f[0] for f in pyclass._fields_] == _struct_fields(cname)


def test_null_args_rejected_without_gpu():
    lib = _lib.lib()
    assert lib.pk_paged_relpos_attn(None, None) == _lib.PK_ERR_INVALID
    assert "NULL" in _lib.last_error()
    assert lib.pk_kv_append(None, None) == _lib.PK_ERR_INVALID
    assert lib.pk_kv_gather(None, None) == _lib.PK_ERR_INVALID
    assert lib.pk_streaming_mask(None, None) == _lib.PK_ERR_INVALID
    assert lib.pk_conv_step(None, None) == _lib.PK_ERR_INVALID
    assert lib.pk_fe_step(None, None) == _lib.PK_ERR_INVALID
    assert lib.pk_subsample(None, None) == _lib.PK_ERR_INVALID
    assert lib.pk_rnnt_greedy_step(None, None) == _lib.PK_ERR_INVALID
    assert lib.pk_hbm_read_probe(None, 16, None, 0, None, None, None) == _lib.PK_ERR_INVALID


def test_read_probe_args_validated_before_launch():
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    addr = (ctypes.addressof(buf) + 15) & ~15  # 16-byte aligned, never dereferenced on a failed check
    assert L.pk_hbm_read_probe(addr, 24, addr, 1, None, None, None) == _lib.PK_ERR_INVALID  # not a multiple of 16
    assert "multiple of 16" in _lib.last_error()
    assert L.pk_hbm_read_probe(addr, 0, addr, 1, None, None, None) == _lib.PK_ERR_INVALID
    assert L.pk_hbm_read_probe(addr, 16, addr, -1, None, None, None) == _lib.PK_ERR_INVALID
    assert L.pk_hbm_read_probe(addr + 8, 16, addr, 1, None, None, None) == _lib.PK_ERR_INVALID  # misaligned


def test_mask_args_validated_before_launch():
    a = _lib.MaskArgs()
    a.batch, a.chunk, a.left, a.chunk_size = 2, 0, 70, 2
    assert _lib.lib().pk_streaming_mask(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.chunk = 2
    assert _lib.lib().pk_streaming_mask(ctypes.byref(a), None) == _lib.PK_ERR_INVALID  # NULL state


def test_conv_args_validated_before_launch():
    L = _lib.lib()
    a = _lib.ConvArgs()
    a.dtype, a.batch, a.chunk, a.d_model, a.kernel = _lib.DTYPE_F16, 2, 2, 512, 9
    a.num_slots, a.num_layers, a.layer = 4, 3, 0
    assert L.pk_conv_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID  # NULL tensors
    assert "NULL" in _lib.last_error()
    a.d_model = 500  # not a multiple of 8 channels
    assert L.pk_conv_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.d_model, a.layer = 512, 3  # layer out of range
    assert L.pk_conv_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.layer, a.batch = 0, 5  # more streams than slots without a slot map
    assert L.pk_conv_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.batch, a.dtype = 0, 7
    assert L.pk_conv_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID  # unknown dtype


def test_residual_norm_args_validated_before_launch():
    L = _lib.lib()
    a = _lib.ResNormArgs()
    a.dtype, a.rows, a.d_model, a.alpha, a.ln_eps = _lib.DTYPE_F16, 4, 512, 0.5, 1e-5
    a.residual_stride = a.branch_stride = a.residual_out_stride = a.norm_out_stride = 512
    assert L.pk_residual_norm(ctypes.byref(a), None) == _lib.PK_ERR_INVALID  # NULL tensors
    assert "NULL" in _lib.last_error()
    a.d_model = 500  # not a multiple of 8 channels
    assert L.pk_residual_norm(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.d_model = 8192  # past 4096 fp16 channels
    assert L.pk_residual_norm(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.d_model, a.alpha = 512, float("nan")
    assert L.pk_residual_norm(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.alpha, a.rows = 1.0, 0  # nothing to do: no pointer is read
    assert L.pk_residual_norm(ctypes.byref(a), None) == _lib.PK_OK
    a.dtype = 7
    assert L.pk_residual_norm(ctypes.byref(a), None) == _lib.PK_ERR_INVALID  # unknown dtype


def test_struct_sizes_match_the_header_alignment():
    # the per-stream headers are read by the kernels as 32-byte records
    assert ctypes.sizeof(_lib.FeStream) == 32 and ctypes.sizeof(_lib.SubStream) == 32


def test_front_end_args_validated_before_launch():
    L = _lib.lib()
    a = _lib.FeArgs()
    a.batch, a.n_fft, a.win_length, a.hop, a.n_mels = 4, 512, 400, 160, 80
    a.ring_size, a.mel_ring_rows, a.num_slots, a.max_new, a.max_frames = 8192, 32, 4, 2560, 16
    a.samples_stride, a.pcm_dtype = 2560, _lib.PCM_S16
    assert L.pk_fe_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID  # NULL tensors
    assert "NULL" in _lib.last_error()
    a.n_fft = 400
    assert L.pk_fe_step(ctypes.byref(a), None) == _lib.PK_ERR_UNSUPPORTED
    a.n_fft, a.ring_size = 512, 8000  # not a power of two
    assert L.pk_fe_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.ring_size, a.max_frames = 8192, 33  # more frames than the mel ring holds
    assert L.pk_fe_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.max_frames, a.n_mels = 16, 129
    assert L.pk_fe_step(ctypes.byref(a), None) == _lib.PK_ERR_UNSUPPORTED
    a.n_mels, a.win_length = 80, 401  # n_fft - win odd
    assert L.pk_fe_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID

    s = _lib.SubArgs()
    s.dtype, s.batch, s.n_mels, s.channels, s.feat_slots, s.feat_rows, s.feat_ring = _lib.DTYPE_F16, 4, 80, 256, 4, 32, 1
    s.out_rows, s.max_out = 8, 2
    assert L.pk_subsample(ctypes.byref(s), None) == _lib.PK_ERR_INVALID  # NULL tensors
    s.channels = 96
    assert L.pk_subsample(ctypes.byref(s), None) == _lib.PK_ERR_UNSUPPORTED
    s.channels, s.feat_rows = 256, 30  # a ring needs a power of two
    assert L.pk_subsample(ctypes.byref(s), None) == _lib.PK_ERR_INVALID
    s.feat_rows, s.dtype = 32, 9
    assert L.pk_subsample(ctypes.byref(s), None) == _lib.PK_ERR_INVALID


def test_rnnt_args_validated_before_launch():
    L = _lib.lib()
    a = _lib.RnntArgs()
    a.dtype, a.batch, a.num_slots, a.layers, a.hidden, a.joint = _lib.DTYPE_F16, 4, 8, 1, 640, 640
    a.vocab1, a.blank, a.max_symbols, a.max_frames = 1027, 1026, 5, 2
    assert L.pk_rnnt_greedy_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID  # NULL tensors
    assert "NULL" in _lib.last_error()
    a.hidden = 512
    assert L.pk_rnnt_greedy_step(ctypes.byref(a), None) == _lib.PK_ERR_UNSUPPORTED
    a.hidden, a.blank = 640, 1027  # blank outside the vocabulary
    assert L.pk_rnnt_greedy_step(ctypes.byref(a), None) == _lib.PK_ERR_INVALID
    a.blank, a.joint = 1026, 600  # joint not a multiple of 64
    assert L.pk_rnnt_greedy_step(ctypes.byref(a), None) == _lib.PK_ERR_UNSUPPORTED
    # workspace: per-stream words 128 x (4 + 2 x 17 tiles of 64 vocabulary rows), two
    # stream lists and their counts, rounded to 256 bytes; then the new h of every
    # stream and layer
    assert L.pk_rnnt_workspace_bytes(_lib.DTYPE_F16, 128, 1027, 1, 640) == 20736 + 128 * 640 * 2
    assert L.pk_rnnt_workspace_bytes(_lib.DTYPE_F32, 1, 1025, 2, 640) == 256 + 2 * 640 * 4


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """With the HIP library absent, the product path raises instead of falling
    back to anything else: the page pool, the cache and the kernel wrappers all
    go through lib()."""
    import torch

    from parakeet_amd import _lib, ops
    from parakeet_amd.modules.cache import ModelCache
    from parakeet_amd.pool import PagePool

    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libparakeet_paged.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        PagePool(2, 16, 70, 2)
    with pytest.raises(RuntimeError, match="missing"):
        ModelCache(1, (70, 1), 64, 9, batch_size=2)
    # host tensors are refused before the library is even looked up
    with pytest.raises(RuntimeError, match="no CPU implementation|missing"):
        ops.streaming_mask(torch.zeros(2, dtype=torch.int64), torch.zeros(2, dtype=torch.int64), 2, chunk=2, left=70, chunk_size=2)
    x = torch.zeros(2, 8, dtype=torch.float16)
    w = torch.ones(8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        ops.residual_norm(x, x, w, w, alpha=0.5)
    with pytest.raises(ValueError, match="must match"):
        ops.residual_norm(x, x[:, :4], w, w)
