"""CPU: the C-ABI library loads, exports every symbol include/dsa_amd.h
declares, and rejects bad arguments before touching a GPU; the Python layer
keeps the reference's error classes.  No kernel is launched here."""
from __future__ import annotations

import ctypes
import math
import os
import re

import pytest
import torch

import _dsa_lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsa_amd.h")


CPU_HEADER = os.path.join(ROOT, "include", "dsa_cpu.h")


def declared_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[A-Za-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    names = declared_functions()
    assert len(names) >= 7, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in dsa_amd.h but not exported"


def test_cpu_library_exports_match_its_header():
    """libdsa_cpu.so (include/dsa_cpu.h): every declared symbol exported,
    nothing else exported under dsa_."""
    import subprocess

    lib = L.cpu_lib()
    names = declared_functions(CPU_HEADER)
    assert names == ["dsa_cpu_isa", "dsa_cpu_last_error", "dsa_cpu_topk_threshold"], names
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", L.CPU_LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if " T dsa_" in ln})
    assert exported == names


def test_export_list_matches_header():
    """Every exported dsa_* function is declared in the header too."""
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if " T dsa_" in ln})
    assert exported == declared_functions()


def test_version_and_limits():
    lib = L.lib()
    assert b"gfx950" in lib.dsa_version()
    assert lib.dsa_fused_max_T() == 2048


def _rc(fn, *args):
    rc = fn(*args)
    return rc, L.lib().dsa_last_error().decode()


FAKE = 0x1000  # never dereferenced: validation fails first


def test_topk_rejects_bad_arguments():
    f = L.lib().dsa_topk_threshold
    cases = [
        ((FAKE, 4, 16, 16, 0, 0, FAKE, None, None), "k must be > 0"),
        ((FAKE, 4, 16, 16, 17, 0, FAKE, None, None), "k must be <= N"),
        ((FAKE, 4, 16, 8, 2, 0, FAKE, None, None), "ld"),
        ((FAKE, -1, 16, 16, 2, 0, FAKE, None, None), "negative"),
        ((FAKE, 6, 16, 16, 2, 4, FAKE, None, None), "multiple"),
        ((FAKE, 4, 16, 16, 2, 32, FAKE, None, None), "causal_T"),
        ((None, 4, 16, 16, 2, 0, FAKE, None, None), "null"),
        ((FAKE, 1, 1 << 31, 1 << 31, 2, 0, FAKE, None, None), "2^31"),
    ]
    for args, needle in cases:
        rc, msg = _rc(f, *args)
        assert rc == L.DSA_EINVAL, (args, rc, msg)
        assert needle in msg, (needle, msg)
    # zero rows is a no-op, not an error
    assert f(None, 0, 16, 16, 2, 0, None, None, None) == L.DSA_OK


def test_indexer_rejects_bad_arguments():
    f = L.lib().dsa_indexer_scores
    ok = (FAKE, FAKE, FAKE, L.DSA_F32, 2, 64, 4, 32, FAKE, 64, 1, None)
    assert _rc(f, *ok[:4], 2, 64, 4, 32, FAKE, 32, 1, None)[0] == L.DSA_EINVAL       # ld < T
    assert _rc(f, *ok[:3], 7, *ok[4:])[0] == L.DSA_EINVAL                              # dtype
    assert _rc(f, *ok[:6], 0, *ok[7:])[0] == L.DSA_EINVAL                              # HI
    assert _rc(f, *ok[:7], 24, *ok[8:])[0] == L.DSA_EUNSUPPORTED                       # DI
    assert _rc(f, FAKE, FAKE, FAKE, L.DSA_BF16, 2, 64, 4, 16, FAKE, 64, 1, None)[0] == L.DSA_EUNSUPPORTED
    assert _rc(f, FAKE + 4, *ok[1:])[0] == L.DSA_EINVAL                                # alignment
    assert _rc(f, None, *ok[1:])[0] == L.DSA_EINVAL                                    # null
    assert f(*ok[:4], 0, *ok[5:]) == L.DSA_OK                                          # B = 0


def test_indexer_strided_rejects_bad_strides():
    f = L.lib().dsa_indexer_scores_strided
    ok = [FAKE, FAKE, FAKE, L.DSA_F32, 2, 64, 4, 32, 132, 132, 132, FAKE, 64, 1, None]
    a = list(ok); a[4] = 0
    assert f(*a) == L.DSA_OK                                         # B = 0, strides fine
    a = list(ok); a[8] = 120
    assert _rc(f, *a)[0] == L.DSA_EINVAL                             # ldq < HI*DI
    a = list(ok); a[9] = 16
    assert _rc(f, *a)[0] == L.DSA_EINVAL                             # ldk < DI
    a = list(ok); a[10] = 3
    assert _rc(f, *a)[0] == L.DSA_EINVAL                             # ldw < HI
    a = list(ok); a[8] = 130
    rc, msg = _rc(f, *a)
    assert rc == L.DSA_EINVAL and "16 bytes" in msg                  # ldq not 16-byte multiple
    a = list(ok); a[3] = L.DSA_BF16; a[8] = a[9] = a[10] = 136
    a[4] = 0
    assert f(*a) == L.DSA_OK                                         # 272-byte rows


def test_fp8_is_indexer_only():
    """DSA_FP8 (e4m3 q_idx/k_idx, fp32 w) is accepted by the indexer for
    DI in {64,128,256} while the q tile fits LDS; attention and the fused
    kernel reject it as an unknown dtype."""
    f = L.lib().dsa_indexer_scores
    fp8 = (FAKE, FAKE, FAKE, L.DSA_FP8)
    assert f(*fp8, 0, 64, 4, 128, FAKE, 64, 1, None) == L.DSA_OK                       # B = 0
    assert _rc(f, *fp8, 2, 64, 4, 32, FAKE, 64, 1, None)[0] == L.DSA_EUNSUPPORTED      # DI 32
    assert _rc(f, *fp8, 2, 64, 256, 256, FAKE, 64, 1, None)[0] == L.DSA_EUNSUPPORTED   # LDS
    assert f(*fp8, 0, 64, 128, 256, FAKE, 64, 1, None) == L.DSA_OK                     # fits
    assert f(*fp8, 0, 64, 156, 256, FAKE, 64, 1, None) == L.DSA_OK                     # 39 groups
    assert _rc(f, *fp8, 2, 64, 160, 256, FAKE, 64, 1, None)[0] == L.DSA_EUNSUPPORTED   # 40 groups
    a = [FAKE, 64, FAKE, FAKE, FAKE, FAKE, L.DSA_FP8, 2, 64, 4, 32, 32, 0.17, FAKE, None]
    assert _rc(L.lib().dsa_sparse_attn_threshold, *a)[0] == L.DSA_EINVAL
    assert _rc(L.lib().dsa_sparse_attn_threshold_tiled, *a)[0] == L.DSA_EINVAL
    a = [FAKE] * 6 + [L.DSA_FP8, 2, 64, 4, 128, 4, 32, 32, 8, 0.17, FAKE, None]
    rc, msg = _rc(L.lib().dsa_fused_forward, *a)
    assert rc == L.DSA_EINVAL and "fp8" in msg


def test_fp8_scaled_entry_checks():
    """dsa_indexer_scores_fp8_scaled: the fp8 indexer's checks, scales 4-byte
    aligned, null scales allowed."""
    f = L.lib().dsa_indexer_scores_fp8_scaled
    assert f(FAKE, FAKE, FAKE, None, None, 0, 64, 4, 128, FAKE, 64, 1, None) == L.DSA_OK
    assert _rc(f, FAKE, FAKE, FAKE, None, None, 2, 64, 4, 32, FAKE, 64, 1, None)[0] == \
        L.DSA_EUNSUPPORTED                                               # fp8 needs DI >= 64
    rc, msg = _rc(f, FAKE, FAKE, FAKE, FAKE + 2, None, 2, 64, 4, 128, FAKE, 64, 1, None)
    assert rc == L.DSA_EINVAL and "aligned" in msg
    assert _rc(f, FAKE, FAKE, FAKE, None, None, 2, 64, 4, 128, FAKE, 32, 1, None)[0] == \
        L.DSA_EINVAL                                                     # ld < T


def test_sparse_attn_rejects_bad_arguments():
    f = L.lib().dsa_sparse_attn_threshold
    base = [FAKE, 64, FAKE, FAKE, FAKE, FAKE, L.DSA_F32, 2, 64, 4, 32, 32, 0.17, FAKE, None]

    def call(**kw):
        a = list(base)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return _rc(f, *a)

    assert call(a9=3)[0] == L.DSA_EINVAL                 # HQ not a power of 2
    assert call(a10=24)[0] == L.DSA_EINVAL               # DQ not a power of 2
    assert call(a1=32)[0] == L.DSA_EINVAL                # ld < T
    assert call(a12=float("nan"))[0] == L.DSA_EINVAL     # scale
    assert call(a0=None)[0] == L.DSA_EINVAL              # null scores
    assert call(a9=128, a10=1, a11=1)[0] == L.DSA_EUNSUPPORTED   # HQ > 64 lanes per head
    assert call(a7=0)[0] == L.DSA_OK


def test_sparse_attn_workspace_entries_check_arguments():
    """The _ws forms validate like the plain ones, refuse a negative
    workspace size, and accept none (B = 0: nothing launched)."""
    for f, staged in ((L.lib().dsa_sparse_attn_threshold_ws, False),
                      (L.lib().dsa_sparse_attn_threshold_staged_ws, True)):
        def call(ws=None, nws=0, **kw):
            a = [FAKE, 4096, FAKE, FAKE, FAKE, FAKE, L.DSA_F32, 2, 4096, 8, 64, 64, 0.125, FAKE,
                 ws, nws, None]
            for i, v in kw.items():
                a[int(i[1:])] = v
            return _rc(f, *a)

        assert call(a1=32)[0] == L.DSA_EINVAL                # ld < T
        assert call(a12=float("inf"))[0] == L.DSA_EINVAL     # scale
        assert call(nws=-1)[0] == L.DSA_EINVAL               # negative workspace size
        assert call(a7=0)[0] == L.DSA_OK                     # B = 0
        assert call(a7=0, ws=FAKE, nws=1 << 20)[0] == L.DSA_OK
        if staged:  # the staged kernel's own shape rule
            assert call(a9=4, a10=32, a11=32)[0] == L.DSA_EUNSUPPORTED


def test_sparse_attn_workspace_bytes_zero_where_unused():
    """No workspace for shapes the staged kernel does not take (16-bit rows
    of 512 at T = 4096 go to the tile kernel, rows of 128 to the gathers,
    T below 3072 stays on the gathers), for bad arguments, and for B = 0."""
    f = L.lib().dsa_sparse_attn_workspace_bytes
    assert f(0, L.DSA_BF16, 1, 4096, 8, 64, 64, 4096) == 0
    assert f(0, L.DSA_F32, 4, 4096, 4, 32, 32, 4096) == 0
    assert f(0, L.DSA_F32, 1, 2048, 8, 64, 64, 2048) == 0
    assert f(0, L.DSA_F32, 0, 4096, 8, 64, 64, 4096) == 0
    assert f(1, L.DSA_F32, 1, 4096, 8, 64, 64, 100) == 0     # ld < T
    assert f(1, 9, 1, 4096, 8, 64, 64, 4096) == 0            # unknown dtype
    assert f(1, L.DSA_F32, 1, 4096, 4, 32, 32, 4096) == 0    # not a staged shape


def test_sparse_attn_accepts_wide_rows():
    """Rows wider than one wave's registers are accepted (head chunks, or the
    tile kernel for 16-bit D in {64,128}); a single head wider than a wave
    holds is not.  B = 0: validation only, nothing launched."""
    f = L.lib().dsa_sparse_attn_threshold

    def rc(dtype, HQ, DQ, DV, B=0, T=512):
        return _rc(f, FAKE, T, FAKE, FAKE, FAKE, FAKE, dtype, B, T, HQ, DQ, DV, 0.1, FAKE, None)

    assert rc(L.DSA_F32, 16, 128, 128)[0] == L.DSA_OK
    assert rc(L.DSA_F32, 4, 512, 512)[0] == L.DSA_OK
    assert rc(L.DSA_F32, 32, 64, 128)[0] == L.DSA_OK
    assert rc(L.DSA_BF16, 128, 128, 128)[0] == L.DSA_OK
    assert rc(L.DSA_BF16, 16, 256, 256)[0] == L.DSA_OK
    assert rc(L.DSA_F16, 64, 64, 64)[0] == L.DSA_OK
    assert rc(L.DSA_F32, 1, 2048, 2048)[0] == L.DSA_EUNSUPPORTED     # one head > 1024 fp32
    assert rc(L.DSA_BF16, 1, 4096, 4096)[0] == L.DSA_EUNSUPPORTED    # one head > 2048 16-bit


def test_tiled_rejects_rows_past_4gib():
    """The tile kernel's DMA offsets are 32-bit bytes within a batch element:
    T*HQ*D*2 >= 4 GiB is refused before any HIP call."""
    f = L.lib().dsa_sparse_attn_threshold_tiled
    T = 1 << 20
    rc, msg = _rc(f, FAKE, T, FAKE, FAKE, FAKE, FAKE, L.DSA_BF16, 1, T, 16, 128, 128, 0.1,
                  FAKE, None)
    assert rc == L.DSA_EINVAL and "4 GiB" in msg, (rc, msg)
    # the gather entry applies the same bound
    rc, msg = _rc(L.lib().dsa_sparse_attn_threshold, FAKE, T, FAKE, FAKE, FAKE, FAKE,
                  L.DSA_BF16, 1, T, 16, 128, 128, 0.1, FAKE, None)
    assert rc == L.DSA_EINVAL and "4 GiB" in msg, (rc, msg)
    # just under the bound is accepted (B = 0: nothing launched)
    assert f(FAKE, T, FAKE, FAKE, FAKE, FAKE, L.DSA_BF16, 0, T, 8, 128, 128, 0.1, FAKE,
             None) == L.DSA_OK


def test_topk_threshold_mask_checks():
    """The select-plus-bitmask entry checks k, the row and mask widths, the
    row count, null pointers and the mask's alignment before any HIP call;
    B = 0 launches nothing."""
    tm = L.lib().dsa_topk_threshold_mask
    ok = [FAKE, 2, 300, 300, 10, FAKE, FAKE, 5, None]

    def rc(**kw):
        a = list(ok)
        for k, v in kw.items():
            a[int(k[1:])] = v
        return _rc(tm, *a)[0]

    assert rc(a4=0) == L.DSA_EINVAL               # k = 0
    assert rc(a4=301) == L.DSA_EINVAL             # k > T
    assert rc(a3=299) == L.DSA_EINVAL             # ld < T
    assert rc(a7=4) == L.DSA_EINVAL               # ldm < ceil(T/64)
    assert rc(a1=-1) == L.DSA_EINVAL              # negative B
    assert rc(a1=1 << 30, a2=4, a3=4, a4=1, a7=1) == L.DSA_EINVAL  # B*T >= 2^31
    assert rc(a0=None) == L.DSA_EINVAL            # null scores
    assert rc(a6=None) == L.DSA_EINVAL            # null mask
    assert rc(a6=FAKE + 4) == L.DSA_EINVAL        # misaligned mask
    assert tm(FAKE, 0, 300, 300, 10, FAKE, FAKE, 5, None) == L.DSA_OK


def test_selection_mask_and_mask_attention_checks():
    """Bitmask entry points: row width, dtype/shape coverage and the 32-bit
    mask-row offsets are checked before any HIP call; B = 0 launches
    nothing."""
    sm = L.lib().dsa_selection_mask
    assert _rc(sm, FAKE, 300, FAKE, 2, 300, FAKE, 4, None)[0] == L.DSA_EINVAL     # ldm < 5
    assert _rc(sm, FAKE, 299, FAKE, 2, 300, FAKE, 5, None)[0] == L.DSA_EINVAL     # ld < T
    assert _rc(sm, None, 300, FAKE, 2, 300, FAKE, 5, None)[0] == L.DSA_EINVAL     # null
    assert _rc(sm, FAKE, 300, FAKE, 2, 300, FAKE + 4, 5, None)[0] == L.DSA_EINVAL  # misaligned
    assert sm(FAKE, 300, FAKE, 0, 300, FAKE, 5, None) == L.DSA_OK
    am = L.lib().dsa_sparse_attn_mask
    ok = [FAKE, 5, FAKE, FAKE, FAKE, L.DSA_BF16, 1, 300, 4, 64, 64, 0.125, FAKE, None]

    def call(**kw):
        a = list(ok)
        for k, v in kw.items():
            a[int(k[1:])] = v
        return _rc(am, *a)

    assert call(a5=L.DSA_F32)[0] == L.DSA_EUNSUPPORTED        # fp32
    assert call(a9=32, a10=32)[0] == L.DSA_EUNSUPPORTED       # D = 32
    assert call(a9=64, a10=128)[0] == L.DSA_EUNSUPPORTED      # DQ != DV
    assert call(a1=4)[0] == L.DSA_EINVAL                      # ldm < ceil(T/64)
    assert call(a1=1 << 21)[0] == L.DSA_EINVAL                # mask rows past 32-bit offsets
    assert call(a0=FAKE + 4)[0] == L.DSA_EINVAL               # mask misaligned
    assert call(a11=math.inf)[0] == L.DSA_EINVAL              # scale
    assert call(a6=0)[0] == L.DSA_OK                          # B = 0


def test_noalloc_entry_checks():
    """dsa_sparse_attn_mask_noalloc: inputs whose bitmask exceeds the static
    scratch (B*T*ceil(T/64) > 2^22 words) and uncovered shapes are refused
    before any HIP call; B = 0 launches nothing."""
    f = L.lib().dsa_sparse_attn_mask_noalloc
    T = 16384
    ok = [FAKE, T, FAKE, FAKE, FAKE, FAKE, L.DSA_BF16, 1, T, 16, 128, 128, 0.1, FAKE, None]
    a = list(ok)
    a[7] = 2                                            # 2 x 16384 x 256 words
    rc, msg = _rc(f, *a)
    assert rc == L.DSA_EINVAL and "static scratch" in msg, (rc, msg)
    a = list(ok)
    a[6] = L.DSA_F32
    assert _rc(f, *a)[0] == L.DSA_EUNSUPPORTED
    a = list(ok)
    a[1] = T - 1                                        # ld < T
    assert _rc(f, *a)[0] == L.DSA_EINVAL
    a = list(ok)
    a[7] = 0
    assert f(*a) == L.DSA_OK


def test_mask_path_rule():
    """dsa_sparse_attn_uses_mask: the shapes dsa_sparse_attn_threshold runs on
    the tile kernel (16-bit, DQ = DV in {64, 128}; T >= 4096 or heads too
    wide to gather)."""
    u = L.lib().dsa_sparse_attn_uses_mask
    assert u(L.DSA_BF16, 16384, 16, 128, 128) == 1
    assert u(L.DSA_F16, 4096, 4, 64, 64) == 1
    assert u(L.DSA_BF16, 4095, 4, 64, 64) == 0
    assert u(L.DSA_BF16, 512, 128, 128, 128) == 1        # 16 K wide rows: tiles at any T
    assert u(L.DSA_F32, 16384, 16, 128, 128) == 0
    assert u(L.DSA_BF16, 16384, 16, 64, 128) == 0
    assert u(L.DSA_BF16, 16384, 16, 32, 32) == 0
    assert u(99, 16384, 16, 128, 128) == 0


def test_fused_rejects_bad_arguments():
    f = L.lib().dsa_fused_forward
    base = [FAKE] * 6 + [L.DSA_F32, 2, 64, 4, 32, 4, 32, 32, 8, 0.17, FAKE, None]
    a = list(base); a[8] = 4096
    assert _rc(f, *a)[0] == L.DSA_EUNSUPPORTED           # T above the fused limit
    a = list(base); a[14] = 0
    assert _rc(f, *a)[0] == L.DSA_EINVAL                 # top_k < 1
    a = list(base); a[10] = 24
    assert _rc(f, *a)[0] == L.DSA_EUNSUPPORTED           # DI


def test_status_mapping():
    with pytest.raises(AssertionError):
        L.check(L.DSA_EINVAL, "x")
    with pytest.raises(L.DSAUnsupported):
        L.check(L.DSA_EUNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        L.check(L.DSA_EHIP, "x")


# ---------------------------------------------------------------------------
# Python drop-ins keep the reference's checks and error classes (CPU tensors:
# they must fail before any kernel launch).
# ---------------------------------------------------------------------------
def test_topk_threshold_contract_errors():
    from topk_threshold import topk_threshold

    x = torch.randn(4, 16)
    with pytest.raises(RuntimeError, match="contiguous"):
        topk_threshold(x.t(), 2)
    with pytest.raises(RuntimeError, match="fp32"):
        topk_threshold(x.double(), 2)
    with pytest.raises(RuntimeError, match="k must be <= N"):
        topk_threshold(x, 17)
    # a CPU tensor is the reference extension's own contract: the host library
    assert torch.equal(topk_threshold(x, 2), x.topk(2, -1).values[..., -1:])


def test_dsa_asserts_match_reference():
    import dsa_attention as D

    def mk(T=32, HI=4, DI=32, HQ=4, D_=32):
        return (torch.zeros(1, T, HI, DI), torch.zeros(1, T, DI), torch.zeros(1, T, HI),
                torch.zeros(1, T, HQ, D_), torch.zeros(1, T, HQ, D_), torch.zeros(1, T, HQ, D_))

    with pytest.raises(AssertionError, match="power of 2"):
        D.dsa_attention_triton(*mk(T=24), top_k=8, BLOCK_S=8)
    with pytest.raises(AssertionError, match="power of 2"):
        D.dsa_attention_triton(*mk(), top_k=6)
    with pytest.raises(AssertionError, match="divisible"):
        D.dsa_attention_triton(*mk(T=16), top_k=8, BLOCK_S=32)
    with pytest.raises(AssertionError):
        D.dsa_attention_split_triton(*mk(), top_k=64)
    with pytest.raises(AssertionError, match="power of 2"):
        D.sparse_attention_with_threshold_triton(torch.zeros(1, 24, 24), torch.zeros(1, 24, 1),
                                                 *mk(T=24)[3:])
    # valid shapes on CPU tensors: rejected as non-GPU input, no launch
    with pytest.raises(AssertionError, match="GPU"):
        D.dsa_attention_triton(*mk(), top_k=8)


def test_indexer_asserts_match_reference():
    from lightning_indexer import indexer_scores_triton

    with pytest.raises(AssertionError):
        indexer_scores_triton(torch.zeros(1, 8, 2, 16), torch.zeros(1, 8, 16), torch.zeros(1, 8, 2))


def test_staged_entry_score_limit():
    """dsa_sparse_attn_threshold_staged addresses one batch element's score
    rows with 32-bit offsets: T*ld*4 >= 2^31 is refused before any HIP call
    (the threshold entry point takes the gathers there); B = 0 launches
    nothing."""
    f = L.lib().dsa_sparse_attn_threshold_staged
    T = 16384
    ok = [FAKE, T, FAKE, FAKE, FAKE, FAKE, L.DSA_F32, 1, T, 8, 64, 64, 0.125, FAKE, None]
    a = list(ok)
    a[1] = 2 * T                                         # 16384 x 32768 x 4 = 2^31 bytes
    rc, msg = _rc(f, *a)
    assert rc == L.DSA_EUNSUPPORTED and "2^31" in msg, (rc, msg)
    a = list(ok)
    a[7] = 0
    assert f(*a) == L.DSA_OK
