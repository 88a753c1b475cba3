"""The oracle's rint quantizers (Q/K codes, int4 activations), its floor(x / s + 1/2) quantizer on rotated rows and
the fp16 rounding points of SwiGLU, the sigmoid gate, situ and modulate, each against exact rational rounding or
float64 closed forms (tests/oracle_pins.py describes each check)."""
import pytest

import oracle
import oracle_pins


@pytest.mark.parametrize("name", sorted(oracle_pins.CHECKS))
def test_oracle_pin(name):
    assert oracle_pins.CHECKS[name](oracle.lib()) == []
