"""The pins of tests/oracle_pins.py see the mistakes they are meant to see: each case copies oracle/rda_oracle.c into a
temporary directory, plants one plausible mistake by a textual substitution (the substituted text must occur exactly
once), builds the copy with the oracle's own compiler flags and checks that the matching pin reports it. The
oracle itself is never modified; the mutants live and die in the test's temporary directory."""
import os
import re
import subprocess

import pytest

import oracle
import oracle_pins

SRC = os.path.join(os.path.dirname(oracle.__file__), "rda_oracle.c")


def oracle_cflags():
    """CFLAGS of oracle/Makefile, so that a mutant differs from the oracle only by its planted mistake."""
    with open(os.path.join(os.path.dirname(oracle.__file__), "Makefile")) as f:
        return re.search(r"^CFLAGS\s*=\s*(.*)$", f.read(), re.M).group(1).split()


# (case, pin that must fail, text of the oracle, its mistaken replacement)
MUTANTS = [
    ("qk_codes_round_half_up", "rint", "(int8_t)(int)rintf(h2f(x[r * ld + d]) / s)", "(int8_t)(int)floorf(h2f(x[r * ld + d]) / s + 0.5f)"),
    ("qk_scale_floor", "rint", "float s = fmaxf(mx / 127.0f, 1e-30f);\n        scale[r] = s;", "float s = fmaxf(mx / 127.0f, 1e-20f);\n        scale[r] = s;"),
    ("qk_reciprocal_product", "rint", "rintf(h2f(x[r * ld + d]) / s)", "rintf(h2f(x[r * ld + d]) * (1.0f / s))"),
    ("int4_round_half_up", "i4", "float f = rintf(y[k] / s);", "float f = floorf(y[k] / s + 0.5f);"),
    ("int4_scale_floor", "i4", "float s = fmaxf(mx, 1e-10f) / 7.0f;", "float s = fmaxf(mx / 7.0f, 1e-10f);"),
    ("int8_round_half_even", "i8_rot", "float f = floorf(y[k] / s + 0.5f);", "float f = rintf(y[k] / s);"),
    ("swiglu_single_rounding", "swiglu", "return r16(r16(gate / (1.0f + orc_expf(-gate))) * up);", "return r16((gate / (1.0f + orc_expf(-gate))) * up);"),
    ("sigmoid_gate_single_rounding", "sigmoid_gate", "return r16(x * r16(1.0f / (1.0f + orc_expf(-gate))));",
     "return r16(x * (1.0f / (1.0f + orc_expf(-gate))));"),
    ("situ_rounded_sigmoid", "situ", "float sigmoid = 1.0f / (1.0f + orc_exp2f(-1.442695041f * gate));",
     "float sigmoid = r16(1.0f / (1.0f + orc_exp2f(-1.442695041f * gate)));"),
    ("modulate_middle_rounding_dropped", "modulate", "return r16(r16(r16(x * rstd * (w + 1.0f)) * s) + t);",
     "return r16(r16(x * rstd * (w + 1.0f)) * s + t);"),
    ("epilogue_scales_multiplied_first", "epilogue", "float y = (float)acc[(size_t)m * N + n] * as[m] * ws[n];",
     "float y = (float)acc[(size_t)m * N + n] * (as[m] * ws[n]);"),
    ("epilogue_bias_fused", "epilogue", "if (bias) y = y + h2f(bias[n]);",
     "if (bias) y = fmaf((float)acc[(size_t)m * N + n] * as[m], ws[n], h2f(bias[n]));"),
    ("residual_inner_rounding_dropped", "gated_residual", "h = f2h(res + r16(gate * h2f(h)));",
     "h = f2h(res + gate * h2f(h));"),
    ("residual_gate_row_index", "gated_residual", "gate = h2f(G[(size_t)(m / L) * N + n]);",
     "gate = h2f(G[(size_t)(m % L) * N + n]);"),
    ("rope_in_double", "rope", "float a = fmaf(m[1], x1, m[0] * x0), c = fmaf(m[3], x1, m[2] * x0);",
     "float a = (float)((double)m[1] * x1 + (double)m[0] * x0), c = (float)((double)m[3] * x1 + (double)m[2] * x0);"),
    ("rope_separate_roundings", "rope", "float a = fmaf(m[1], x1, m[0] * x0), c = fmaf(m[3], x1, m[2] * x0);",
     "float a = m[1] * x1 + m[0] * x0, c = m[3] * x1 + m[2] * x0;"),
    ("rope_matrix_transposed", "rope", "float a = fmaf(m[1], x1, m[0] * x0), c = fmaf(m[3], x1, m[2] * x0);",
     "float a = fmaf(m[2], x1, m[0] * x0), c = fmaf(m[3], x1, m[1] * x0);"),
    ("w4a8_scale_before_sum", "w4a8_epilogue", "float t = y * as[m];", "float t = r16(y) * as[m];"),
]


@pytest.mark.parametrize("case,pin,text,mistake", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_pin_sees_planted_mistake(tmp_path, case, pin, text, mistake):
    with open(SRC) as f:
        src = f.read()
    assert src.count(text) == 1, f"{case}: the text to mutate must occur exactly once in rda_oracle.c"
    path = tmp_path / "rda_oracle_mutant.c"
    path.write_text(src.replace(text, mistake))
    so = tmp_path / f"lib_{case}.so"
    subprocess.run(["gcc", *oracle_cflags(), "-o", str(so), str(path), "-lm"], check=True)
    failures = oracle_pins.CHECKS[pin](oracle.load(str(so)))
    assert failures, f"{case}: the {pin} pin did not see the planted mistake"
