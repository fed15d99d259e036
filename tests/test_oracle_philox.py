"""Pins oracle/philox.py against the Random123 KATs and rocRAND's engine."""
import json
import os

import numpy as np

from oracle.philox import philox4x32_10, philox_uniforms, philox_words, words_to_uniform

GOLD = os.path.join(os.path.dirname(__file__), "golden", "philox_kat.json")


def _load():
    with open(GOLD) as f:
        return json.load(f)


def test_random123_kat():
    for case in _load()["random123"]:
        ctr = np.array([int(x, 16) for x in case["ctr"]], np.uint32)
        key = np.array([int(x, 16) for x in case["key"]], np.uint32)
        out = philox4x32_10(ctr, key)
        assert [f"{int(x):08x}" for x in out] == case["out"]


def test_rocrand_engine_words():
    for case in _load()["rocrand"]:
        w = philox_words(case["seed"], case["stream"], case["offset"], len(case["words"]))
        assert [int(x) for x in w] == case["words"], case


def test_uniform_mapping_exact():
    w = np.array([0, 255, 256, 0xFFFFFFFF, 0x80000000], np.uint32)
    u = words_to_uniform(w)
    assert u.dtype == np.float32
    assert list(u) == [0.0, 0.0, 2.0 ** -24, (2 ** 24 - 1) * 2.0 ** -24, 0.5]
    assert np.all(u < 1.0)


def test_offsets_are_a_sliding_window():
    a = philox_uniforms(7, 3, 0, 40)
    b = philox_uniforms(7, 3, 13, 20)
    assert np.array_equal(a[13:33], b)
    c = philox_uniforms(7, 4, 0, 40)
    assert not np.array_equal(a, c)
