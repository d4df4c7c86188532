"""CPU-only checks of the product's host side: layout helpers and the synthetic
generator against the oracle, the C ABI library (loads, exports every symbol the
header declares, host entry points and argument validation -- nothing that
launches a kernel), and the vLLM plugin surface (op schemas, _C functions and
argument names, config API, create_weights)."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from oracle import wlq_oracle as O
from qwen_wlqfastshot_helen_beta_amd import ABI_HEADER, formats, load_abi, synth

# ---------------------------------------------------------------- formats / synth


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_formats_match_oracle(bits):
    rng = np.random.default_rng(bits)
    N, K = 7, 157
    codes = rng.integers(0, 1 << bits, (N, K)).astype(np.uint8)
    q, wpr = formats.pack_indices_row_aligned(codes, bits)
    q_o, wpr_o = O.pack_row_aligned(codes, bits)
    assert wpr == wpr_o == formats.words_per_row(K, bits)
    assert np.array_equal(q.view(np.uint32), q_o.view(np.uint32))
    qc = formats.pack_indices_continuous(codes, bits)
    assert np.array_equal(qc.view(np.uint32), O.pack_continuous(codes, bits).view(np.uint32))
    assert np.array_equal(formats.unpack_indices_continuous(qc, N, K, bits), codes)
    assert formats.chunk_width(bits) == O.chunk_width(bits)
    assert formats.num_chunks(K, bits) == O.num_chunks(K, bits)


def test_e5m2_and_csr_match_oracle():
    u16 = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(formats.fp16_to_e5m2_u8(u16.view(np.float16)), O.fp16_bits_to_e5m2(u16))
    rng = np.random.default_rng(5)
    mask = rng.random((9, 1300)) < 0.02
    vals = rng.integers(0, 256, mask.sum()).astype(np.uint8)
    for chunk in (512, 640):
        off, cols, v = formats.build_chunk_csr(mask, vals, chunk)
        off_o, cols_o, v_o = O.build_chunk_csr(mask, vals, chunk)
        assert np.array_equal(off, off_o) and np.array_equal(cols, cols_o) and np.array_equal(v, v_o)


def test_metalog_luts_follow_normal_quantiles():
    from scipy.stats import norm

    rng = np.random.default_rng(0)
    luts = synth.metalog_luts(rng, 4000, 4, sigma=0.02).astype(np.float64)
    assert np.all(np.diff(luts, axis=1) >= 0)  # sorted
    # averaged over many fits, entry j sits near the N(0, 0.02) quantile at (j + 1/2) / 16
    target = norm.ppf((np.arange(16) + 0.5) / 16) * 0.02
    assert np.max(np.abs(luts.mean(axis=0) - target)) < 0.003
    # the projector reproduces an exact 4-term metalog: fitting samples on its own curve
    y = (np.arange(1, 129) - 0.5) / 128
    coef = np.array([0.01, 0.003, -0.002, 0.004])
    samples = synth.metalog_basis(y, 4) @ coef
    P = synth.metalog_lut_projector(4)
    yq = (np.arange(16) + 0.5) / 16
    assert np.allclose(P @ samples, synth.metalog_basis(yq, 4) @ coef, atol=1e-12)


def test_synth_layer_invariants():
    L = synth.make_layer(N=50, K=700, bits=4, group_size=128, rank=4, density=0.02, seed=3, heavy_frac=0.2,
                         heavy_mult=10.0)
    assert L.nnz == round(0.02 * 50 * 700)
    rows = np.repeat(np.arange(50), np.diff(L.offsets[:, [0, -1]], axis=1).ravel())
    counts = np.bincount(rows, minlength=50)
    assert counts.max() >= 5 * np.median(counts[counts > 0])  # heavy rows present
    assert np.all(np.diff(L.offsets.ravel()) >= 0) and L.offsets[0, 0] == 0 and L.offsets[-1, -1] == L.nnz
    assert L.cols.max() < 512
    W = O.dequant(L.q, L.lut, L.N, L.K, 4, L.offsets, L.cols, L.vals, group_size=128)
    assert W.shape == (50, 700) and W.dtype == np.float16
    # headline bytes: codes + LUT + 3 bytes per outlier + offsets
    assert L.headline_bytes() == L.q.nbytes + L.lut.nbytes + 3 * L.nnz + L.offsets.nbytes


def test_merge_layers_matches_oracle_merge():
    a = synth.make_layer(N=20, K=256, bits=4, group_size=128, rank=2, density=0.03, seed=1)
    b = synth.make_layer(N=12, K=256, bits=4, group_size=128, rank=3, density=0.03, seed=2)
    m = synth.merge_layers([a, b])
    Wa = O.dequant(a.q, a.lut, a.N, a.K, 4, a.offsets, a.cols, a.vals, group_size=128)
    Wb = O.dequant(b.q, b.lut, b.N, b.K, 4, b.offsets, b.cols, b.vals, group_size=128)
    Wm = O.dequant(m.q, m.lut, m.N, m.K, 4, m.offsets, m.cols, m.vals, group_size=128)
    assert np.array_equal(Wm.view(np.uint16), np.concatenate([Wa, Wb]).view(np.uint16))
    A, B, _ = O.merge_dora([a.A, b.A], [a.B, b.B], [None, None])
    assert np.array_equal(m.A.astype(np.float64), A) and np.array_equal(m.B.astype(np.float64), B)


# ---------------------------------------------------------------- C ABI (no kernel launches)


def _header_functions():
    text = open(ABI_HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wlq_[a-z0-9_]+)\s*\(", text)))


def test_abi_exports_every_declared_symbol():
    lib = load_abi()
    names = _header_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), f"libwlq_hip.so does not export {n}"
    assert lib.wlq_abi_version() == 5
    assert lib.wlq_status_string(4) == b"WLQ_ERR_CAPACITY" or b"capacity" in lib.wlq_status_string(4).lower()


def test_abi_workspace_status_without_counter_area():
    """Host-side argument handling of the workspace status/reset entry points (no GPU call):
    a null workspace or one below the 16 KiB counter area has no counters to check."""
    lib = load_abi()
    assert lib.wlq_workspace_status(None, 0, None) == 0
    assert lib.wlq_workspace_status(None, 1 << 20, None) == 0
    assert lib.wlq_workspace_reset(None, 1 << 20, None) == 1  # WLQ_ERR_NULL_POINTER
    assert b"non-null" in lib.wlq_last_error()
    assert b"hand-off" in lib.wlq_status_string(7)


def test_abi_prepared_bytes():
    """Size of the prepared layout (host query, no GPU): 256-byte aligned parts
    codes | planes | gcol | delta | patch-list starts | patches; 0 for formats without one."""
    lib = load_abi()
    a = lambda v: (v + 255) // 256 * 256  # noqa: E731
    for N, K, G, nnz in ((37888, 3584, 128, 678960), (77, 1000, 32, 100), (16, 512, 0, 0), (5, 8, 128, 1)):
        T, S = -(-N // 16), -(-K // 128)
        ng = 1 if G == 0 or G >= K else -(-K // G)
        want = a(T * S * 1024) + a(T * ng * 512) + a(nnz * 2) + a(nnz * 4) + a((T * S + 1) * 4) + a(nnz * 4)
        assert lib.wlq_prepared_bytes(N, K, 4, G, nnz) == want, (N, K, G)
        # 3-bit: the same layout (codes as 4-bit nibbles, LUTs padded to 16); groups of >= 40 columns
        assert lib.wlq_prepared_bytes(N, K, 3, G, nnz) == (0 if 0 < G < 40 and G < K else want), (N, K, G)
    assert lib.wlq_prepared_bytes(64, 640, 2, 64, 0) == 0     # 2-bit
    assert lib.wlq_prepared_bytes(64, 1024, 1, 128, 0) == 0   # 1-bit
    assert lib.wlq_prepared_bytes(64, 960, 4, 48, 0) == 0     # group not a multiple of 32
    assert lib.wlq_prepared_bytes(64, 1001, 4, 128, 0) == 0   # K % 8 != 0
    assert lib.wlq_prepared_bytes(64, 70000, 4, 128, 0) == 0  # columns beyond 16 bits


def test_abi_host_helpers_match_oracle():
    lib = load_abi()
    for bits in (1, 2, 3, 4):
        for K in (1, 31, 896, 3584, 18944):
            assert lib.wlq_words_per_row(K, bits) == O.words_per_row(K, bits)
        assert lib.wlq_chunk_width(bits) == O.chunk_width(bits)
    # continuous -> row-aligned repack
    rng = np.random.default_rng(9)
    for bits in (1, 2, 3, 4):
        N, K = 5, 77
        codes = rng.integers(0, 1 << bits, (N, K)).astype(np.uint8)
        src = O.pack_continuous(codes, bits).view(np.uint32)
        wpr = O.words_per_row(K, bits)
        dst = np.zeros(N * wpr, dtype=np.uint32)
        st = lib.wlq_repack_row_aligned(src.ctypes.data, src.size, N, K, bits, dst.ctypes.data, dst.size)
        assert st == 0, lib.wlq_last_error()
        assert np.array_equal(dst, O.pack_row_aligned(codes, bits)[0].view(np.uint32))
        # a destination that is too small is refused
        st = lib.wlq_repack_row_aligned(src.ctypes.data, src.size, N, K, bits, dst.ctypes.data, dst.size - 1)
        assert st == 4
    # rows of whole, unpadded words (K a multiple of the codes per word, words per row a
    # multiple of 4): the word-copy path, against the oracle's repack, incl. 3-bit words whose
    # unused top bits are set in the source and a source one word short
    for bits, K in ((4, 3584), (4, 64), (2, 256), (1, 128), (3, 1280)):
        N = 6
        codes = rng.integers(0, 1 << bits, (N, K)).astype(np.uint8)
        src = O.pack_continuous(codes, bits).view(np.uint32).copy()
        wpr = O.words_per_row(K, bits)
        assert K % O.symbols_per_word(bits) == 0 and K // O.symbols_per_word(bits) == wpr
        if bits == 3:
            src |= np.uint32(0xC0000000)
        want = O.pack_row_aligned(codes, bits)[0].view(np.uint32)
        dst = np.full(N * wpr, 0xFFFFFFFF, dtype=np.uint32)
        assert lib.wlq_repack_row_aligned(src.ctypes.data, src.size, N, K, bits, dst.ctypes.data, dst.size) == 0
        assert np.array_equal(dst, want), (bits, K)
        dst[:] = 0xFFFFFFFF
        assert lib.wlq_repack_row_aligned(src.ctypes.data, src.size - 1, N, K, bits, dst.ctypes.data, dst.size) == 0
        want_short = want.copy()
        want_short[-1] = 0
        assert np.array_equal(dst, want_short), (bits, K)


def test_abi_ef_decoder_matches_oracle():
    lib = load_abi()
    rng = np.random.default_rng(11)
    N, K, T, C = 45, 70, 32, 512
    mask = rng.random((N, K)) < 0.05
    meta, stream = O.ef_encode(mask, T)
    meta = np.ascontiguousarray(meta, dtype=np.int64)
    stream = np.ascontiguousarray(stream, dtype=np.uint32)
    total = lib.wlq_ef_total(meta.ctypes.data, meta.shape[0])
    assert total == mask.sum()
    nch = O.num_chunks(K, 4)
    off = np.zeros((N, nch + 1), dtype=np.int32)
    cols = np.zeros(max(total, 1), dtype=np.uint16)
    nnz = ctypes.c_int64(0)
    st = lib.wlq_ef_decode_chunk_csr(meta.ctypes.data, meta.shape[0], stream.ctypes.data, stream.size, N, K, T, C,
                                     off.ctypes.data, cols.ctypes.data, cols.size, ctypes.byref(nnz))
    assert st == 0, lib.wlq_last_error()
    off_o, cols_o = O.ef_decode_to_chunk_csr(meta, stream, N, K, T, C)
    assert np.array_equal(off, off_o) and np.array_equal(cols[:nnz.value], cols_o)


def test_abi_validation_before_launch():
    """Bad arguments are refused with a status and a message, before any HIP call."""
    lib = load_abi()
    buf = np.zeros(4096, dtype=np.uint8)
    p = buf.ctypes.data
    p16 = (p + 15) & ~15
    # unsupported width
    st = lib.wlq_gemv(p16, p16, p16, p16, None, None, None, None, None, None, None, 1.0, 0, 8, 32, 5, 0, None, 0,
                      None)
    assert st == 3 and lib.wlq_last_error()
    # null codes
    st = lib.wlq_gemv(None, p16, p16, p16, None, None, None, None, None, None, None, 1.0, 0, 8, 32, 4, 0, None, 0,
                      None)
    assert st == 1
    # words_per_row inconsistent with K and bits
    st = lib.wlq_gemm(p16, p16, p16, p16, 2, 8, 32, 4, 3, 0, None, None, None, None, None, None, None, 1.0, 0, None, 0,
                      None)
    assert st == 2
    # group size not a multiple of 32
    st = lib.wlq_gemm(p16, p16, p16, p16, 2, 8, 256, 4, 32, 48, None, None, None, None, None, None, None, 1.0, 0, None,
                      0, None)
    assert st == 3
    # misaligned code pointer
    st = lib.wlq_gemv(p16 + 4, p16, p16, p16, None, None, None, None, None, None, None, 1.0, 0, 8, 32, 4, 0, None, 0,
                      None)
    assert st == 2


# ---------------------------------------------------------------- plugin surface


def test_op_schemas_match_reference():
    import qwen_wlqfastshot_helen_beta_amd.vllm_wlq  # noqa: F401  registers the ops

    # the alias set name of the mutated `out` is generated by torch.library (a, a3, ...)
    gemv = re.sub(r"\(a\d*!\)", "(a!)", str(torch.ops.wlq_fastShot.gemv.default._schema))
    gemm = re.sub(r"\(a\d*!\)", "(a!)", str(torch.ops.wlq_fastShot.gemm.default._schema))
    assert gemv.startswith("wlq_fastShot::gemv(Tensor q_packed, Tensor lut_c, Tensor x, Tensor(a!) out, SymInt N, "
                           "SymInt K, SymInt bits, Tensor? chunk_offsets=None, Tensor? chunk_cols=None, "
                           "Tensor? chunk_vals=None, Tensor? lora_B=None, Tensor? lora_h=None, "
                           "Tensor? dora_gamma=None, float lora_scale=1."), gemv
    assert gemm.startswith("wlq_fastShot::gemm(Tensor X, Tensor q_packed, Tensor lut_c, Tensor(a!) out, SymInt N, "
                           "SymInt K, SymInt bits, SymInt words_per_row, Tensor? chunk_offsets"), gemm
    # lora_H before lora_B in gemm (reference order), trailing defaulted extensions only
    assert gemm.index("lora_H") < gemm.index("lora_B")
    assert gemv.endswith("float lora_scale=1., SymInt group_size=0, Tensor? lora_A=None, "
                         "Tensor? prepared=None) -> ()")
    assert gemm.endswith("float lora_scale=1., SymInt group_size=0, Tensor? lora_A=None, "
                         "Tensor? prepared=None) -> ()")


def test_c_extension_functions():
    from qwen_wlqfastshot_helen_beta_amd.vllm_wlq import _C

    for name in ("gemv_forward", "gemm_forward", "dequant_w0", "init_workspaces", "decode_ef_to_chunk_csr",
                 "repack_q_indices_row_aligned", "prepare_layer"):
        assert hasattr(_C, name), name
    doc = _C.dequant_w0.__doc__
    for arg in ("q_packed", "lut_c", "W_out", "N", "K", "bits", "words_per_row", "chunk_offsets", "chunk_cols",
                "chunk_vals"):
        assert arg in doc, arg
    # host functions run without a GPU
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, (3, 50)).astype(np.uint8)
    raw = torch.from_numpy(O.pack_continuous(codes, 4).view(np.int32))
    q, wpr = _C.repack_q_indices_row_aligned(raw, 3, 50, 4)
    assert wpr == O.words_per_row(50, 4)
    assert np.array_equal(q.numpy().view(np.uint32), O.pack_row_aligned(codes, 4)[0].view(np.uint32))
    mask = rng.random((10, 40)) < 0.1
    meta, stream = O.ef_encode(mask, 32)
    off, cols = _C.decode_ef_to_chunk_csr(torch.from_numpy(np.asarray(meta, np.int64)),
                                          torch.from_numpy(np.asarray(stream, np.uint32).view(np.int32)), 10, 40, 32,
                                          512)
    off_o, cols_o = O.ef_decode_to_chunk_csr(meta, stream, 10, 40, 32, 512)
    assert np.array_equal(off.numpy(), off_o) and np.array_equal(cols.numpy().view(np.uint16), cols_o)


def test_quant_config_api():
    from qwen_wlqfastshot_helen_beta_amd.vllm_wlq import WLQFastShotConfig, WLQLinearMethod

    cfg = WLQFastShotConfig.from_config({"bits": 3, "use_dora": False})
    assert cfg.get_name() == "wlq_fastShot"
    assert WLQFastShotConfig.get_min_capability() == 80
    assert WLQFastShotConfig.get_config_filenames() == ["/config.json"]
    assert torch.float16 in cfg.get_supported_act_dtypes()
    assert cfg.bits == 3 and cfg.chunk_m == 640
    assert cfg.get_scaled_act_names() == []
    assert isinstance(WLQLinearMethod(cfg), WLQLinearMethod)


def test_create_weights_parameters():
    from qwen_wlqfastshot_helen_beta_amd.vllm_wlq import WLQFastShotConfig, WLQLinearMethod

    m = WLQLinearMethod(WLQFastShotConfig(bits=4))
    layer = torch.nn.Module()
    m.create_weights(layer, 256, [64, 32], 256, 96, torch.float16)
    names = {n for n, _ in layer.named_parameters()}
    # the checkpoint tensors the reference's loader registers (vllm_wlq/linear_method.py:376-411)
    assert names == {"bits", "ef_bitstream", "ef_tile_meta", "ef_tile_size", "fp8_outliers", "is_quantized", "lut_c",
                     "orig_shape", "outlier_mask", "outlier_mask_1bit", "outlier_values", "outliers", "q_packed",
                     "weight"}, names


def test_bench_refuses_multi_gpu_runs():
    """bench.py measures one GPU: --gpus N > 1 (or a torchrun world) exits with a message, before
    touching a device."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in r.stdout + r.stderr
