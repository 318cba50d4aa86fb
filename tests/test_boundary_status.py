"""The host's reading of a boundary's device status words (no GPU): the states that leave a
valid outcome, the ones that raise, and how the rows were moved."""
import os
import re

import pytest

from gstar_evict import _native as N
from gstar_evict.compaction import OVERFLOW_WORD, outcome

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _words(state=0, protected=4608, width=28160, count=32768, leftover=1, relocation=0, overflow=0):
    w = [0] * 16
    w[:9] = [state, protected, width, count, leftover, 0, protected, protected, relocation]
    w[OVERFLOW_WORD] = overflow
    return w


def test_evicted_boundary_and_its_relocation_path():
    got = outcome(_words())
    assert got == {"state": N.BOUNDARY_EVICTED, "protected": 4608, "count": 32768, "leftover": 1,
                   "relocation": "single pass"}
    assert outcome(_words(relocation=N.RELOCATION_SCRATCH))["relocation"] == "scratch"


def test_deferred_boundary_passes_through():
    got = outcome(_words(state=N.BOUNDARY_DEFERRED, protected=5000, width=0, count=0, leftover=0))
    assert got["state"] == N.BOUNDARY_DEFERRED and got["protected"] == 5000


@pytest.mark.parametrize("words,message", [
    (_words(state=N.BOUNDARY_ERR_RELOCATE), "timed out after its first phase"),
    (_words(state=N.BOUNDARY_ERR_HEADS), "protected positions differ between heads"),
    (_words(overflow=1), "queue overflowed"),
])
def test_states_without_a_valid_outcome_raise(words, message):
    with pytest.raises(RuntimeError, match=message):
        outcome(words)


def test_status_words_match_the_header():
    """gse_boundary_status has nine int32 fields, `relocation` last; the flush's overflow word
    sits past them in the 16-word status buffer; the relocation and state codes agree."""
    text = open(os.path.join(ROOT, "include", "gstar_evict.h")).read()
    body = re.search(r"typedef struct \{(.*?)\} gse_boundary_status;", text, re.S).group(1)
    fields = re.findall(r"int32_t\s+(\w+);", body)
    assert len(fields) == 9 and fields[0] == "state" and fields[-1] == "relocation"
    assert len(fields) <= OVERFLOW_WORD < 16
    codes = dict(re.findall(r"(GSE_(?:RELOCATION|BOUNDARY)_\w+)\s*=\s*(\d+)", text))
    assert int(codes["GSE_RELOCATION_SCRATCH"]) == N.RELOCATION_SCRATCH
    assert int(codes["GSE_RELOCATION_SINGLE_PASS"]) == N.RELOCATION_SINGLE_PASS
    assert int(codes["GSE_BOUNDARY_ERR_RELOCATE"]) == N.BOUNDARY_ERR_RELOCATE
