"""LDS direct loads stay inside their regions, checked on the CPU.

A global_load_lds writes its 64 lanes' bytes at M0 + 16 * lane (dwordx4) or
M0 + 4 * lane (dword) whatever the source address, so an M0 too close to the
end of a region writes past it - into the next table, or past the workgroup's
LDS - and can fault the GPU.  The prefill kernels' sites (pf_expert codes and
tables, sh_gemm codes and scales) depend only on compile-time constants and
are checked by static_asserts in k_prefill.hip (so this file's first test is
that the library built at all from the current sources).  The decode
launches' sites depend on the batch: sf37k_decode_lds_check recomputes the
launch plan's LDS layout on the host (the function the launchers use) and
checks every direct-load span against its region and every region against
the LDS its launch is given, for each batch size 1..16, with and without the
one-token up launch, at the BASELINE shape and the reduced test shapes, at
gfx950's 160 KiB per workgroup and at 64 KiB.  Reference practice: argument
checks before any launch (sf37_cuda.cu:5286-5310)."""
import ctypes as C
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROUTER, SELECT, SHARED, UPSEL = 1, 2, 4, 64


@pytest.fixture(scope="module")
def lib():
    from sf37_amd import hip
    L = hip.lib()
    fn = L.sf37k_decode_lds_check
    fn.restype = C.c_int
    fn.argtypes = [C.c_uint32] * 7 + [C.POINTER(C.c_uint64)]
    return L


def test_prefill_static_asserts_compiled():
    """The library's objects are newer than k_prefill.hip: the static_asserts
    on the direct-load extents held when it was compiled."""
    src = os.path.join(ROOT, "sf37_amd", "csrc", "k_prefill.hip")
    obj = os.path.join(ROOT, "_build", "k_prefill.o")
    so = os.path.join(ROOT, "sf37_amd", "libsf37_hip.so")
    text = open(src).read()
    assert text.count("static_assert(") >= 6 and "stay in their buffer" in text
    if not os.path.exists(obj):
        pytest.skip("no object build here")
    assert os.path.getmtime(obj) >= os.path.getmtime(src) and os.path.getmtime(so) >= os.path.getmtime(obj)


SHAPES = [(288, 8, 4096, 1280), (16, 8, 512, 256), (32, 8, 1024, 512), (288, 3, 4096, 1280),
          (288, 4, 4096, 768), (64, 8, 2048, 512), (288, 8, 4096, 512)]


@pytest.mark.parametrize("E,topk,K,F", SHAPES)
def test_decode_direct_loads_fit(lib, E, topk, K, F):
    ext = (C.c_uint64 * 6)()
    seen_wide = 0
    for max_lds in (163840, 65536):
        for T in range(1, 17):
            for flags in (ROUTER | SELECT | SHARED, ROUTER | SELECT | SHARED | UPSEL, SELECT):
                r = lib.sf37k_decode_lds_check(T, topk, E, K, F, flags, max_lds, ext)
                assert r in (0, -1), (T, flags, max_lds, r, list(ext))
                if r == 0 and ext[0]:
                    seen_wide += 1
                    assert ext[0] <= ext[1] <= max_lds and ext[4] <= ext[5]
                if r == 0 and (flags & SHARED):
                    assert 0 < ext[2] <= ext[3] <= max_lds
                if (E, topk, K, F) == (288, 8, 4096, 1280) and max_lds == 163840:
                    assert r == 0, f"BASELINE shape refused at {T} tokens"
    if K in (2048, 4096):
        assert seen_wide > 0        # the block-pair DMA path was among the plans checked


def test_decode_check_sees_an_overflow(lib):
    """The check has the power to fail: a limit below one tile's span past the
    activations is refused before launch (-1) or reported, never passed."""
    ext = (C.c_uint64 * 6)()
    r = lib.sf37k_decode_lds_check(16, 8, 288, 4096, 1280, SELECT | SHARED, 20000, ext)
    assert r != 0
