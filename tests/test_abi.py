"""CPU checks of the C-ABI boundary: the library loads, exports every
function include/sf37_hip.h declares, and the device exp/sigmoid source
equals the host libm-based sigmoid on every binary32 input."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    from sf37_amd import hip
    L = hip.lib()
    syms = hip.header_symbols()
    assert len(syms) >= 59
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    # every declared function has a ctypes signature in the binding
    assert set(syms) <= set(hip._SIGS), sorted(set(syms) - set(hip._SIGS))


def test_engine_hook_library_exports_its_header():
    """libsf37_engine_moe.so (the engine's SF37_USE_HIP MoE block, a C caller
    of libsf37_hip.so) loads and exports what include/sf37_engine_moe.h
    declares."""
    import ctypes as C
    import re
    text = open(os.path.join(ROOT, "include", "sf37_engine_moe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    syms = sorted(set(re.findall(r"\b(sf37_engine_[a-z0-9_]+)\s*\(", text)))
    assert syms == ["sf37_engine_moe_decode", "sf37_engine_moe_prefill"]
    L = C.CDLL(os.path.join(ROOT, "sf37_amd", "libsf37_engine_moe.so"))
    assert all(hasattr(L, s) for s in syms)


def test_engine_hook_refuses_dense_layers(capfd):
    """Layers 0-2 are dense (sf37.c:2245-2249): the MoE block refuses them
    with a 'dense layer' line before any HIP call, so no GPU is needed."""
    import ctypes as C
    from test_gpu_engine import EngineBufs, EngineLayer
    L = C.CDLL(os.path.join(ROOT, "sf37_amd", "libsf37_engine_moe.so"))
    L.sf37_engine_moe_decode.restype = L.sf37_engine_moe_prefill.restype = C.c_int
    bufs = EngineBufs()
    for il in (0, 1, 2):
        lay = EngineLayer(il=il, n_expert=288, topk=8, embd=4096, expert_ff=1280)
        assert L.sf37_engine_moe_decode(C.byref(lay), C.byref(bufs)) == 0
        assert L.sf37_engine_moe_prefill(C.byref(lay), C.byref(bufs), C.c_uint32(4)) == 0
    err = capfd.readouterr().err
    assert err.count("is a dense layer") == 6, err


def test_reference_entry_points_are_mirrored():
    """Each hot-path entry of the reference interface (sf37_cuda.h) has a
    sf37_hip_ twin with the same name suffix."""
    from sf37_amd import hip
    hot = ["device_count", "print_devices", "init", "cleanup", "synchronize", "memory_info",
           "begin_layer", "end_layer", "set_model_fd", "set_model_map_range", "set_model_map_spans",
           "cache_model_range", "evict_model_cache", "tensor_alloc", "tensor_alloc_managed",
           "tensor_free", "tensor_bytes", "tensor_write", "tensor_read", "tensor_copy", "tensor_fill_f32",
           "rms_norm_weight1_f32", "rms_norm_weight1_bf16", "add_inplace_f32", "swiglu_f32",
           "matvec_q8_0", "matvec_q8_0_pair", "matvec_f32", "matvec_q3_asym", "matvec_q2_asym",
           "router_select", "routed_moe_one", "rms_norm_weight1_bf16_mapped",
           "rms_norm_weight1_bf16_batch_mapped", "matvec_q8_0_mapped", "matmul_q8_0_mapped",
           "matmul_q8_0_pair_mapped", "matvec_q8_0_pair_mapped", "matvec_f32_mapped", "matmul_f32_mapped",
           "matvec_q3_asym_mapped", "matvec_q2_asym_mapped", "router_select_mapped",
           "router_select_batch_mapped", "routed_moe_one_mapped", "routed_moe_batch_mapped",
           "matvec_bf16", "matvec_bf16_mapped", "matmul_bf16_mapped"]
    syms = set(hip.header_symbols())
    assert {"sf37_hip_" + h for h in hot} <= syms


def test_no_device_no_crash():
    """Without a GPU the runtime reports no device instead of failing."""
    from sf37_amd import hip
    assert hip.lib().sf37_hip_device_count() >= -1


def test_device_exp_source_matches_libm_exhaustively(tmp_path):
    exe = tmp_path / "expf_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I", os.path.join(ROOT, "sf37_amd", "csrc"), os.path.join(ROOT, "tests", "host_expf_check.cpp"),
                    "-o", str(exe), "-lpthread"], check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "expf_mismatch 0 sigmoid_mismatch 0" in r.stdout


def test_router_split_plan():
    """The prefill router GEMM's K split (k_router.hip rl_plan): the smallest
    power-of-two slice count up to 16 that gives about three workgroups per
    CU (256 CUs without a device, as on MI355X), only where the slices keep
    K in 64-wide chunks; the workspace is one binary64 partial per slice,
    token and expert, and none where the product runs unsplit."""
    import ctypes as C
    from sf37_amd import hip
    f = hip.lib().sf37k_f32_matmul_part_bytes
    f.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
    f.restype = C.c_uint64
    E = 288
    for k, t, slices in [(4096, 512, 16), (4096, 1100, 8), (4096, 2048, 4), (4096, 4096, 2),
                         (4096, 17, 16), (384, 512, 2), (4096, 40000, 1), (4096, 16, 1),
                         (4000, 512, 1)]:
        want = slices * t * E * 8 if slices > 1 else 0
        assert f(k, E, t) == want, (k, t, slices, f(k, E, t))
