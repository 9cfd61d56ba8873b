"""The C-ABI library (no GPU needed): it loads, exports every entry point that
include/*.h declares, and its host-side validation mirrors the reference's
SamplingParameters::validate (output_head_sampler.rs:56-75)."""
import ctypes as C
import os
import re

import pytest

from yskn_smp import (EINVAL, GUMBEL, INVERSE_CUMULATIVE, InvalidInput, SamplingParameters,
                      load_library)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    syms = set()
    inc = os.path.join(ROOT, "include")
    for f in os.listdir(inc):
        if f.endswith(".h"):
            txt = open(os.path.join(inc, f)).read()
            txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
            syms |= set(re.findall(r"\b(yskn_smp_[a-z_]+)\s*\(", txt))
    return syms


def test_library_exports_every_declared_symbol():
    L = load_library()
    syms = declared_symbols()
    assert len(syms) >= 12
    for s in sorted(syms):
        assert hasattr(L, s), s


def test_version_and_last_error_are_strings():
    L = load_library()
    assert b"gfx950" in L.yskn_smp_version()
    assert isinstance(L.yskn_smp_last_error(), bytes)


def test_from_thousandths_and_defaults_validate():
    p = SamplingParameters.from_thousandths(700, 900, 50)
    assert (p.temperature, p.top_p, p.min_p) == (0.7, 0.9, 0.05)
    SamplingParameters().validate(248_320)
    SamplingParameters(temperature_milli=0).validate(1)   # greedy needs nothing else


@pytest.mark.parametrize("kw", [dict(top_k=0), dict(top_k=21), dict(top_p_milli=0),
                                dict(top_p_milli=1001), dict(min_p_milli=1001), dict(version=1),
                                dict(repetition_penalty=0.0),
                                dict(frequency_penalty=float("inf"))])
def test_invalid_parameters_are_rejected(kw):
    with pytest.raises(InvalidInput) as e:
        SamplingParameters(**kw).validate(248_320)
    assert e.value.code == EINVAL
    assert "invalid input" in str(e.value)


def test_top_k_bounds_against_vocabulary():
    with pytest.raises(InvalidInput):
        SamplingParameters(top_k=20).validate(19)
    SamplingParameters(top_k=19).validate(19)
    # extended top-k: 0 (disabled) and up to V
    SamplingParameters(top_k=0).validate(1000, flags=1)
    SamplingParameters(top_k=1000).validate(1000, flags=1)
    with pytest.raises(InvalidInput):
        SamplingParameters(top_k=1001).validate(1000, flags=1)


def test_both_versions_validate():
    for v in (GUMBEL, INVERSE_CUMULATIVE):
        SamplingParameters(version=v).validate(100)


# SamplingParameters::validate on binary64 fields as they are
# (output_head_sampler.rs:56-75): NaN and infinities fail every range check.
@pytest.mark.parametrize("kw,msg", [
    (dict(temperature=0.0), "temperature"), (dict(temperature=-1.0), "temperature"),
    (dict(temperature=float("nan")), "temperature"), (dict(temperature=float("inf")), "temperature"),
    (dict(top_p=0.0), "top_p"), (dict(top_p=1.0000000000000002), "top_p"),
    (dict(top_p=float("nan")), "top_p"),
    (dict(min_p=-5e-324), "min_p"), (dict(min_p=1.0000000000000002), "min_p"),
    (dict(min_p=float("nan")), "min_p"),
    (dict(top_k=0), "top_k"), (dict(top_k=21), "top_k"),
])
def test_binary64_parameters_follow_the_reference_rules(kw, msg):
    from yskn_smp import SamplingParametersF64
    with pytest.raises(InvalidInput) as e:
        SamplingParametersF64(**kw).validate(248_320)
    assert msg in str(e.value)


def test_binary64_parameters_accept_the_reference_ranges():
    from yskn_smp import SamplingParametersF64
    SamplingParametersF64().validate(248_320)                     # the reference defaults
    SamplingParametersF64(temperature=5e-324, top_p=5e-324, min_p=1.0, top_k=20).validate(20)
    SamplingParametersF64(temperature=0.7123456789, top_p=1.0, min_p=0.0, top_k=1).validate(1)
    # greedy (Sampler::Greedy) carries no sampling parameters to validate
    SamplingParametersF64(temperature=float("nan"), greedy=True).validate(1)
