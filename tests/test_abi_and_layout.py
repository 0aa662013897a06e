"""CPU checks of the product library: the C ABI loads and exports every
declared symbol, the no-device and bad-argument paths return the documented
status codes, and the arithmetic trick and tiled layout the kernels rely on
are exact (emulated here in numpy binary16 arithmetic)."""
import os
import re
import subprocess

import numpy as np
import pytest

import mnb_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mnb.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mnb_[a-z_0-9]+)\s*\(", text)))


def test_header_declarations_match_binding_list():
    assert _declared_symbols() == sorted(mnb_hip.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    L = mnb_hip.load()
    for name in _declared_symbols():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", mnb_hip.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (mnb_[a-z_0-9]+)", out))
    assert set(_declared_symbols()) <= exported
    assert mnb_hip.load().mnb_version() == 1


def test_struct_layouts_match_the_header(tmp_path):
    """The C structs a foreign binding lays out by hand (the ctypes binding
    here; the Java FFM binding's 72-byte mnb_group_item) have the header's
    size and field offsets."""
    import ctypes
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "mnb.h"\n'
                   'int main(void) { printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n", sizeof(mnb_group_item),\n'
                   '  offsetof(mnb_group_item, weight), offsetof(mnb_group_item, M), offsetof(mnb_group_item, x),\n'
                   '  offsetof(mnb_group_item, x_type), offsetof(mnb_group_item, x_elems), offsetof(mnb_group_item, y),\n'
                   '  offsetof(mnb_group_item, y_type), offsetof(mnb_group_item, y_elems), offsetof(mnb_group_item, flags));\n'
                   '  return 0; }\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I" + os.path.dirname(HEADER), "-o", str(exe), str(src)], check=True)
    c = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    G = mnb_hip.GroupItem
    py = [ctypes.sizeof(G)] + [getattr(G, f).offset for f in
                               ("weight", "M", "x", "x_type", "x_elems", "y", "y_type", "y_elems", "flags")]
    assert c == py
    assert c == [72, 0, 8, 16, 24, 32, 40, 48, 56, 64]   # the offsets the Java binding writes


def test_no_device_or_device_path_reports_status():
    import ctypes
    L = mnb_hip.load()
    h = ctypes.c_void_p()
    rc = L.mnb_context_create(0, ctypes.byref(h))
    if rc == mnb_hip.MNB_OK:          # running on a GPU host: nothing to check here
        assert L.mnb_context_destroy(h) == mnb_hip.MNB_OK
        pytest.skip("a device is present")
    assert rc == mnb_hip.MNB_ERR_NO_DEVICE
    assert "device" in mnb_hip.last_error()
    with pytest.raises(mnb_hip.MnbError):
        mnb_hip.Context(0)


def test_null_handles_fail_with_reference_semantics():
    import ctypes
    L = mnb_hip.load()
    out = ctypes.c_void_p()
    q = np.zeros(64, np.uint8)
    s = np.ones(2, np.float32)
    rc = L.mnb_weight_create(None, 2, 64, 32, 4, q.ctypes.data, q.size, s.ctypes.data, mnb_hip.MNB_F32, s.size,
                             None, 0, mnb_hip.MNB_ZP_NONE, 0, ctypes.byref(out))
    assert rc == mnb_hip.MNB_ERR_INVALID_STATE and "Kernel not prepared" in mnb_hip.last_error()
    rc = L.mnb_matmul(None, None, 1, None, 0, 0, None, 0, 0, 0, None)
    assert rc == mnb_hip.MNB_ERR_INVALID_STATE
    with pytest.raises(mnb_hip.IllegalStateException):
        mnb_hip.check(rc)
    assert L.mnb_weight_destroy(None) == mnb_hip.MNB_OK
    assert L.mnb_supports_batch(None) == 0
    assert L.mnb_max_batch_rows() >= 1 << 20


# ---------------------------------------------------------------------------
# numpy emulation of the device arithmetic
# ---------------------------------------------------------------------------

def _h2(u32):
    """uint32 array -> (lo, hi) float16 halves"""
    u = np.asarray(u32, np.uint32)
    return (u & 0xFFFF).astype(np.uint16).view(np.float16), (u >> 16).astype(np.uint16).view(np.float16)


def unpack_q_minus_zp(d, zp):
    """Emulation of mnb_device.h unpack_q_minus_zp on one tiled dword."""
    d = np.uint32(d)
    blo = np.uint32(0x64006400 | (zp * 0x00010001))
    bhi = np.uint32(0x54005400 | ((zp << 4) * 0x00010001))
    lo0, lo1 = _h2(blo)
    hi0, hi1 = _h2(bhi)
    d8 = d >> np.uint32(8)
    sixteenth = np.float16(0.0625)
    out = []
    for word, is_hi in (((d & 0x000F000F) | 0x64006400, False), ((d & 0x00F000F0) | 0x64006400, True),
                        ((d8 & 0x000F000F) | 0x64006400, False), ((d8 & 0x00F000F0) | 0x64006400, True)):
        a, b = _h2(np.uint32(word))
        if is_hi:
            # fused multiply-add: exact product then one rounding; here the
            # product a/16 is exact, so two binary16 steps give the same value
            out += [np.float16(np.float16(a * sixteenth) - hi0), np.float16(np.float16(b * sixteenth) - hi1)]
        else:
            out += [np.float16(a - lo0), np.float16(b - lo1)]
    return np.array(out, np.float16)


def unzip(s):
    t = 0
    for i in range(8):
        nib = (s >> (4 * i)) & 0xF
        pos = 16 + 4 * (i >> 1) if i & 1 else 4 * (i >> 1)
        t |= nib << pos
    return t


def test_nibble_to_fp16_trick_is_exact_for_all_values():
    # every (nibble, zero point) pair at every one of the 8 positions
    for zp in range(16):
        for q in range(16):
            for pos in range(8):
                nat = q << (4 * pos)              # natural order: k_pos = q, others 0
                got = unpack_q_minus_zp(unzip(nat), zp)
                exp = np.array([(q if i == pos else 0) - zp for i in range(8)], np.float16)
                assert np.array_equal(got, exp), (q, zp, pos)


def test_unpack_gives_mfma_operand_order_on_random_words():
    rng = np.random.default_rng(0)
    for _ in range(200):
        ks = rng.integers(0, 16, 8)
        zp = int(rng.integers(0, 16))
        nat = 0
        for i, v in enumerate(ks):
            nat |= int(v) << (4 * i)               # k0 in the low nibble of byte 0, k1 in its high nibble
        got = unpack_q_minus_zp(unzip(nat), zp)
        assert np.array_equal(got, (ks - zp).astype(np.float16))


def tiled_index(N, K, bs, n, k):
    """(dword index in the tiled q buffer, nibble position in natural order)"""
    kb = -(-K // bs)
    ST = -(-(kb * bs) // 128)
    nt, r = divmod(n, 16)
    st, kk = divmod(k, 128)
    j, rem = divmod(kk, 32)
    g, i = divmod(rem, 8)
    lane = g * 16 + r
    return ((nt * ST + st) * 64 + lane) * 4 + j, i


def test_tiled_layout_is_a_bijection_and_loads_are_contiguous():
    N, K, bs = 40, 384, 32
    seen = set()
    for n in range(N):
        for k in range(0, K, 8):
            dw, i = tiled_index(N, K, bs, n, k)
            assert i == 0
            assert dw not in seen
            seen.add(dw)
    # one wave load (64 lanes x 16 bytes) covers one 16x128 tile exactly
    dws = sorted(tiled_index(N, K, bs, n, k)[0] for n in range(16) for k in range(0, 128, 8))
    assert dws == list(range(256))
