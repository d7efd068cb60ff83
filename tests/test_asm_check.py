"""The build's scan of inline-asm MFMAs (raftinfer_amd/asm_check.py) on small
listings whose answer is fixed by counting wait states, and on the built
prefill kernel itself."""
import pathlib

from raftinfer_amd import asm_check
from raftinfer_amd.asm_check import RESULT_WAIT_STATES, asm_mfma_hazards

MFMA = """\t;;#ASMSTART
\ts_nop 1
\tv_mfma_f32_32x32x16_bf16 a[16:31], v[30:33], v[6:9], a[16:31]
\t;;#ASMEND
"""


def test_copy_right_after_an_asm_mfma_is_flagged():
    text = MFMA + "\tv_accvgpr_mov_b32 a2, a17\n"
    hazards = asm_mfma_hazards(text)
    assert len(hazards) == 1 and "a[16:31]" in hazards[0] and "after 0 wait states" in hazards[0]


def test_reads_after_the_drain_or_of_other_registers_pass():
    drained = MFMA + "\ts_nop 7\n\ts_nop 7\n\ts_nop 3\n\tv_accvgpr_read_b32 v0, a16\n"
    assert asm_mfma_hazards(drained) == []
    other = MFMA + "\tv_accvgpr_read_b32 v0, a32\n\tv_accvgpr_mov_b32 a1, a15\n"
    assert asm_mfma_hazards(other) == []


def test_wait_states_are_counted_exactly():
    # s_nop n gives n + 1 wait states; one short of the latency is flagged, the latency is not
    short = MFMA + "\ts_nop 7\n" * 2 + f"\ts_nop {RESULT_WAIT_STATES - 16 - 2}\n" + "\tv_add_f32 v1, a20, v2\n"
    assert len(asm_mfma_hazards(short)) == 1
    enough = MFMA + "\ts_nop 7\n" * 2 + f"\ts_nop {RESULT_WAIT_STATES - 16 - 1}\n" + "\tv_add_f32 v1, a20, v2\n"
    assert asm_mfma_hazards(enough) == []


def test_compiler_mfmas_and_mfma_chains_are_not_flagged():
    # a compiler-placed MFMA (outside ASMSTART/ASMEND) is the compiler's own business, and an
    # accumulator chain is checked by the hardware
    text = "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[4:7], v[8:11], 0\n\tv_accvgpr_read_b32 v0, a0\n"
    text += MFMA + MFMA
    assert asm_mfma_hazards(text) == []


def test_built_prefill_kernel_has_no_hazard():
    s = pathlib.Path(asm_check.__file__).resolve().parent / "_build" / "attention_prefill_mfma.hip.s"
    if not s.exists():
        import pytest
        pytest.skip("the library has not been built here")
    assert asm_mfma_hazards(s.read_text()) == []
