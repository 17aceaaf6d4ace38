"""C-ABI boundary checks that run without a GPU: the library loads, exports
every symbol include/praghip.h declares, its host-side table builder agrees
with the oracle and the closed form, and argument validation rejects bad
plans before any device call."""
import ctypes
import os
import re

import numpy as np
import pytest

import closed_form as cf
import oracle
import praghip
from praghip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    with open(os.path.join(ROOT, "include", "praghip.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(praghip_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    names = header_functions()
    assert len(names) >= 20
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in names:
        assert hasattr(L, name), name
    # the Python binding declares a signature for every exported entry point
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_library_links_no_oracle():
    with open(_lib.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"orc_" not in blob and b"liboracle" not in blob


@pytest.mark.parametrize("log_n", [4, 10, 12, 14])
def test_tables_match_oracle(log_n):
    n = 1 << log_n
    for q in (cf.LOCKED_PRIMES[0], cf.LOCKED_PRIMES[6], cf.primes_below(50, n, 1)[0], cf.primes_below(54, n, 1)[0]):
        f, i, ninv, psi = praghip.ntt_tables(q, log_n)
        of, oi, on = oracle.ntt_tables(q, log_n)
        assert psi == oracle.minimal_root(q, n)
        np.testing.assert_array_equal(f, of)
        np.testing.assert_array_equal(i, oi)
        np.testing.assert_array_equal(ninv, on)


def test_locked_psi_values(golden_dir):
    import json
    with open(os.path.join(golden_dir, "primes.json")) as fh:
        psis = [int(x) for x in json.load(fh)["psi_16384"]]
    for q, want in zip(cf.LOCKED_PRIMES, psis):
        assert praghip.ntt_tables(q, 14)[3] == want


def test_plan_validation_before_device():
    with pytest.raises(praghip.PraghipError) as e:
        praghip.NttBatch([1152921504599080963], 14)  # not prime
    assert e.value.code == _lib.E_CONTEXT and "E_NTT_CONTEXT" in e.value.text
    with pytest.raises(praghip.PraghipError) as e:
        praghip.NttBatch([cf.LOCKED_PRIMES[0]], 15)
    assert e.value.code == _lib.E_SHAPE
    with pytest.raises(praghip.PraghipError) as e:
        praghip.NttBatch([101], 4)  # 101 != 1 mod 32
    assert e.value.code == _lib.E_CONTEXT
    f, i, n, _ = praghip.ntt_tables(cf.LOCKED_PRIMES[1], 10)
    f[5, 1] ^= 1  # corrupted quotient
    with pytest.raises(praghip.PraghipError) as e:
        praghip.NttBatch([cf.LOCKED_PRIMES[1]], 10, tables=(f[None], i[None], n[None]))
    assert e.value.code == _lib.E_CONTEXT
    with pytest.raises(praghip.PraghipError) as e:
        praghip.Switch(cf.LOCKED_PRIMES, 14, dnum=7)
    assert e.value.code == _lib.E_SHAPE
    with pytest.raises(praghip.PraghipError) as e:
        praghip.Switch(cf.LOCKED_PRIMES, 14, dnum=6, element=4)
    assert e.value.code == _lib.E_ARGUMENT


def seal_switch_tables(q, log_n):
    """The arrays the reference's Switch::initialize(q, f, r, ni, invp, keys)
    receives (keyswitch/seal_adapter.cpp:24-41): SEAL's root-power tables from
    the oracle, and inv_q_last_mod_q computed here from the definition
    (q[L]^-1 mod q_i with its Shoup quotient floor(w 2^64 / q_i))."""
    t = oracle.Tables(q, log_n)
    invp = []
    for qi in q[:-1]:
        w = pow(q[-1] % qi, qi - 2, qi)
        assert w * q[-1] % qi == 1
        invp += [w, (w << 64) // qi]
    return {"fwd": t.fwd, "inv": t.inv, "invn": t.invn, "invp": np.array(invp, dtype=np.uint64)}


def test_switch_takes_and_checks_seal_tables():
    """Switch::initialize's tables: the right ones pass validation (the call
    then stops only at the device check here), and one corrupted operand or
    quotient in any of them is E_NTT_CONTEXT before any device call."""
    q, log_n = cf.LOCKED_PRIMES, 10
    good = seal_switch_tables(q, log_n)
    if praghip.device_count() == 0:
        with pytest.raises(praghip.PraghipError) as e:
            praghip.Switch(q, log_n, dnum=6, tables=good)
        assert e.value.code == _lib.E_DEVICE
    for name, idx in (("fwd", (3, 77, 1)), ("inv", (6, 5, 0)), ("invn", (2, 1)), ("invp", (9,))):
        bad = {k: v.copy() for k, v in good.items()}
        bad[name][idx] ^= 1
        with pytest.raises(praghip.PraghipError) as e:
            praghip.Switch(q, log_n, dnum=6, tables=bad)
        assert e.value.code == _lib.E_CONTEXT and "E_NTT_CONTEXT" in e.value.text, name
    with pytest.raises(ValueError):
        praghip.Switch(q, log_n, dnum=6, tables={"forward": good["fwd"]})


def test_no_device_here_is_reported():
    if praghip.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(praghip.PraghipError) as e:
        praghip.NttBatch([cf.LOCKED_PRIMES[0]], 14)
    assert e.value.code == _lib.E_DEVICE and "E_GFX950_REQUIRED" in e.value.text


def test_device_binding_requires_both_variables(monkeypatch):
    """The UUID + PCI binding of ntt.cu:86-90: an unset or empty variable is
    E_PHASE_DEVICE_BINDING before any device is looked at."""
    monkeypatch.delenv("PRAG_ENC0_GPU_UUID", raising=False)
    monkeypatch.setenv("PRAG_ENC0_GPU_PCI", "0000:c1:00.0")
    with pytest.raises(praghip.PraghipError) as e:
        praghip.bind_device()
    assert e.value.code == _lib.E_DEVICE and e.value.text == "E_PHASE_DEVICE_BINDING"
    monkeypatch.setenv("PRAG_ENC0_GPU_UUID", "")
    with pytest.raises(praghip.PraghipError) as e:
        praghip.bind_device()
    assert e.value.text == "E_PHASE_DEVICE_BINDING"
    monkeypatch.setenv("PRAG_SILU_GPU_UUID", "GPU-0000000000000000")
    monkeypatch.delenv("PRAG_SILU_GPU_PCI", raising=False)
    with pytest.raises(praghip.PraghipError) as e:
        praghip.bind_device(uuid_var="PRAG_SILU_GPU_UUID", pci_var="PRAG_SILU_GPU_PCI")
    assert e.value.text == "E_PHASE_DEVICE_BINDING"
    with pytest.raises(praghip.PraghipError) as e:
        praghip.bind_device(uuid="GPU-0000000000000000", pci=None)
    assert e.value.text == "E_PHASE_DEVICE_BINDING"


def test_device_binding_without_a_match():
    """No gfx950 device has this identity (none at all without a GPU):
    E_GFX950_REQUIRED, and the index stays -1."""
    import ctypes
    out = ctypes.c_int(7)
    rc = _lib.lib().praghip_device_bind(b"GPU-not-a-device", b"ffff:ff:1f.7", ctypes.byref(out))
    assert rc == _lib.E_DEVICE and out.value == -1
    assert _lib.lib().praghip_last_error().decode().startswith("E_GFX950_REQUIRED")
    buf = ctypes.create_string_buffer(64)
    assert _lib.lib().praghip_device_identity(0, buf, 39, buf, 64) == _lib.E_ARGUMENT


def test_share_entry_points_validate_before_device():
    """The ring ops, lift, dyadic MAC, local dot and batched GEMM reject bad
    arguments before any device call (fake, aligned addresses are never touched)."""
    import ctypes

    import numpy as np
    L = _lib.lib()
    A = 1 << 20  # 16-byte aligned fake device address
    q = np.array(cf.LOCKED_PRIMES[:2], dtype=np.uint64)

    def code(rc):
        return rc, L.praghip_last_error().decode()

    assert code(L.praghip_ring_add(0, A, A, A, 8, 0, None)) == (_lib.E_ARGUMENT, "E_SHARE_MASK")
    assert code(L.praghip_ring_add(0, A + 8, A, A, 8, 59, None)) == (_lib.E_ARGUMENT, "E_SHARE_ALIGNMENT")
    assert code(L.praghip_ring_add(0, None, A, A, 8, 59, None)) == (_lib.E_ARGUMENT, "E_NULL")
    assert L.praghip_ring_add(0, None, None, None, 0, 59, None) == _lib.OK  # empty is a no-op
    assert code(L.praghip_ring_scale(0, A, 3, A, 8, 65, None)) == (_lib.E_ARGUMENT, "E_SHARE_MASK")
    assert code(L.praghip_ring_layout(0, A, 0, A, A, 4, None)) == (_lib.E_SHAPE, "E_CUDA_SHAPE")
    assert code(L.praghip_ring_sum_rows(0, A, A, 4, 0, 59, None)) == (_lib.E_SHAPE, "E_CUDA_SHAPE")
    assert code(L.praghip_lift59(0, A, A, 1, 12, 5000, q.ctypes.data, 2, None)) == (_lib.E_SHAPE, "E_LIFT_SHAPE")
    bad_q = np.array([cf.LOCKED_PRIMES[0], 4], dtype=np.uint64)  # even modulus
    assert code(L.praghip_lift59(0, A, A, 1, 12, 0, bad_q.ctypes.data, 2, None)) == (_lib.E_SHAPE, "E_LIFT_SHAPE")
    assert code(L.praghip_dyadic_mac(0, A, A, A, 0, 2, 12, 2, q.ctypes.data, 2, None)) == (_lib.E_SHAPE,
                                                                                           "E_DYADIC_SHAPE")
    delta = np.array([q[0], 1], dtype=np.uint64)  # Delta_0 not below q_0
    assert code(L.praghip_local_dot_scale(0, A, A, 16, 1, delta.ctypes.data, 5, q.ctypes.data, 2, A, A, None)) == (
        _lib.E_CANONICAL, "E_LOCAL_DELTA")
    assert code(L.praghip_local_dot_scale(0, A, A, 16, 1, delta.ctypes.data, 1 << 59, q.ctypes.data, 2, A, A,
                                          None)) == (_lib.E_SHAPE, "E_LOCAL_SHAPE")
    assert L.praghip_local_dot_workspace_words(3) == 3 * 256
    # the allocation-free variant: its scratch holds 64 slots; argument checks first
    assert code(L.praghip_local_dot_scale_noalloc(0, A, A, 16, 65, delta.ctypes.data, 5, q.ctypes.data, 2, A,
                                                  None)) == (_lib.E_SHAPE, "E_LOCAL_NOALLOC_SLOTS: at most 64 slots")
    assert code(L.praghip_local_dot_scale_noalloc(0, A, None, 16, 1, delta.ctypes.data, 5, q.ctypes.data, 2, A,
                                                  None)) == (_lib.E_ARGUMENT, "E_NULL")
    assert code(L.praghip_local_dot_scale_noalloc(0, A, A, 16, 1, delta.ctypes.data, 5, q.ctypes.data, 2, A,
                                                  None)) == (_lib.E_CANONICAL, "E_LOCAL_DELTA")
    assert L.praghip_local_dot_scale_noalloc(0, None, None, 16, 0, None, 5, None, 0, None, None) == _lib.OK
    descs = (_lib.GemmDesc * 2)(_lib.GemmDesc(A, A, None, A, 4, 8, 4, 8, 64), _lib.GemmDesc(A, A, None, A, 4, 8, 4, 16, 64))
    assert code(L.praghip_share_gemm_batch(0, ctypes.cast(descs, ctypes.c_void_p), 2, None)) == (
        _lib.E_ARGUMENT, "E_SHARE_WEIGHT_DTYPE")
    descs[1].w_bits, descs[1].y = 32, A + 4
    assert code(L.praghip_share_gemm_batch(0, ctypes.cast(descs, ctypes.c_void_p), 2, None)) == (
        _lib.E_ARGUMENT, "E_SHARE_ALIGNMENT")
