"""The C ABI without a GPU: libcqhip.so loads, exports every entry point
include/cqhip.h declares, rejects bad packed matrices with the reference's
messages (internal/cq/cq_test.go:561-585), and fails loudly, not by a CPU
fallback, when there is no device."""

import ctypes
import os
import re

import numpy as np
import pytest

import go_whistle_amd as gw
from go_whistle_amd import _lib, synth
from conftest import ROOT, gpu_available


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:cq|kv|nd)_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared("cqhip.h")
    assert len(names) >= 20
    lib = _lib.lib()
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_oracle_exports_its_header():
    from oracle import binding

    text = open(os.path.join(ROOT, "oracle", "oracle.h")).read()
    names = set(re.findall(r"\b(orc_\w+)\s*\(", text))
    lib = binding.lib()
    for n in names:
        assert hasattr(lib, n), n


def test_product_library_does_not_link_the_oracle():
    so = open(_lib.LIB_PATH, "rb").read()
    assert b"orc_" not in so and b"liboracle" not in so


def _new(p, gather=False):
    return gw.cq.Matrix._new(p, gather)


@pytest.mark.parametrize("edit,want", [
    (dict(Bits=3, Width=3), "not supported"),
    (dict(Bits=5), "not supported"),
    (dict(Group=24), "power of two"),
    (dict(Group=4), "power of two"),
    (dict(Out=-1), "bad shape"),
    (dict(In=0), "bad shape"),
    ("cb3", "codebook"),
    ("index", "index"),
    ("norms", "norm"),
])
def test_new_errors_through_the_abi(edit, want):
    g = synth.rng(7)
    good = synth.random_packed(g, 2, 128, 128, 2)
    kw = dict(good.__dict__)
    if edit == "cb3":
        kw["Codebook"] = good.Codebook[:3]
    elif edit == "index":
        kw["Index"] = good.Index[1:]
    elif edit == "norms":
        kw["Norms"] = good.Norms[2:]
    else:
        kw.update(edit)
    with pytest.raises(gw.CQError) as e:
        _new(gw.cq.Packed(**kw))
    assert str(e.value).startswith("cq: ") and want in str(e.value)


def test_no_device_fails_loudly():
    if gpu_available():
        pytest.skip("a device is present")
    p = synth.random_packed(synth.rng(1), 4, 128, 128, 4)
    with pytest.raises(gw.CQDeviceError) as e:
        _new(p)
    assert "no HIP device" in str(e.value)


def test_quantize_rows_misuse_through_the_abi():
    with pytest.raises(gw.CQPanic):
        gw.needle.QuantizeRows(np.zeros(96, np.float32), 96, 40)


def test_noalloc_reorder_refuses_oversize_before_the_device():
    # kv_reorder_noalloc_dev checks its temporaries against its 16 MiB array
    # before any device call: 256 streams x 512 rows x 512 codes exceed it
    from ctypes import c_void_p

    p = c_void_p(256)  # never dereferenced: the size check comes first
    with pytest.raises(gw.CQPanic) as e:
        _lib.check(_lib.lib().kv_reorder_noalloc_dev(p, p, p, p, 256, 512, 512, 64, None))
    assert "16777216" in str(e.value)


@pytest.mark.parametrize("eos,done", [(-1, True), (16384, True), (5, False)])
def test_argmax_eos_misuse_before_the_device(eos, done):
    # nd_argmax_advance_eos_dev rejects a stop token outside the vocabulary
    # and a nil done mask before any device call
    from ctypes import c_void_p

    p = c_void_p(256)  # never dereferenced: the checks come first
    with pytest.raises(gw.CQPanic):
        _lib.check(_lib.lib().nd_argmax_advance_eos_dev(p, p, 4, 16384, p, p, 4, p if done else None, eos, None))
