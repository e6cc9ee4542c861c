"""The library build's m0 guard (triton_llm/_build.py check_m0): kernels
that issue the inline-asm LDS-DMA, which writes m0, must contain no
compiler-generated m0 use.  Checked here on small assembly listings; the
build runs it on every device object."""

import pytest

from triton_llm import _build

DMA = """\t;;#ASMSTART
\ts_mov_b32 m0, s4
\tbuffer_load_dwordx4 v1, s[8:11], 0 offen lds
\t;;#ASMEND
"""


def listing(name, body):
    return f"\t.type\t{name},@function\n{name}:\n{body}\ts_endpgm\n.Lfunc_end0:\n"


def test_dma_kernel_without_compiler_m0_passes():
    text = listing("k_dma", "\tv_mov_b32 v0, 0\n" + DMA + "\ts_waitcnt vmcnt(0)\n")
    assert _build.check_m0(text, "t.hip") == 1


@pytest.mark.parametrize("use", ["\ts_mov_b32 m0, s2\n", "\tv_movrels_b32 v0, v1\n",
                                 "\tbuffer_load_dword v2, s[0:3], 0 offen lds\n"])
def test_compiler_m0_use_in_a_dma_kernel_fails(use):
    # in another basic block of the same kernel, after the asm
    text = listing("k_bad", DMA + ".LBB0_2:\n" + use)
    with pytest.raises(RuntimeError, match="k_bad"):
        _build.check_m0(text, "t.hip")


def test_m0_use_in_a_kernel_without_the_dma_is_allowed():
    text = listing("k_dma", DMA) + listing("k_other", "\ts_mov_b32 m0, -1\n\tds_read_b32 v0, v1\n")
    assert _build.check_m0(text, "t.hip") == 1
