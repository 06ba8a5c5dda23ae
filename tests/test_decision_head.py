"""The config-3 decision head (q35m_letter_logits, the arithmetic q35m_decide applies to the
label rows) against the reference's own known answers for letter_logits
(tests/cua_s1/head.rs:4-30): float64 accumulation, float32 readout, only the first n rows
read, non-finite logits refused. Host-only: no device work, runs without a GPU."""
import numpy as np
import pytest

from qwen3_5_native import hip
from qwen3_5_native import model as QM

BIG = 16_777_216.0  # 2^24: 2^24 + 1 is not a float32


def test_float64_accumulation_and_float32_readout():
    letters = np.array([BIG, 1.0, -BIG, BIG, 1.0, 0.0, np.nan, np.nan, np.nan], np.float32)
    last = np.ones(3, np.float32)
    # row 0 sums to 1 in float64 (0 in float32); row 1 is 2^24 + 1, read out as the float32 2^24;
    # row 2 (NaN) is never read
    assert QM.letter_logits(letters, last, 2).tolist() == [1.0, BIG]
    assert QM.letter_logits(letters, last, 1).tolist() == [1.0]


@pytest.mark.parametrize("letters,last", [([np.finfo(np.float32).max], [2.0]), ([np.nan], [1.0])])
def test_non_finite_logits_are_refused(letters, last):
    with pytest.raises(hip.HipError):
        QM.letter_logits(np.array(letters, np.float32), np.array(last, np.float32), 1)
