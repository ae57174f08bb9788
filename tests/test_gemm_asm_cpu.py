"""The prefill GEMM's generated assembly main loop, emulated on the CPU (tests/gemm_asm_emulator.py).

Every case runs the exact instruction stream that gemm.hip compiles (gen_gemm_asm.py) against an int64 matmul of the
same operands: group counts 1..18 (every entry phase of the six-group unrolled body, one or several loop iterations),
ragged row and column tiles (masked stores), A8 rows and A16 digit-row pairs with the colterm. The emulator also
fails a missing or too weak wait, a copy into LDS still being read, and any access outside its buffer; planted
mistakes in the generator show that it does.
"""
import numpy as np
import pytest

import gemm_asm_emulator as E

G = E.G


@pytest.mark.parametrize("pairs,K,Mrows,N", [
    (False, 128, 256, 128), (False, 256, 256, 128), (False, 384, 200, 128), (False, 512, 256, 100),
    (False, 640, 256, 128), (False, 768, 300, 192), (False, 1664, 256, 64), (False, 2304, 256, 128),
    (True, 768, 256, 128), (True, 1664, 300, 192), (True, 128, 256, 64)])
def test_generated_gemm_matches_int64_matmul(pairs, K, Mrows, N):
    T, ref = E.emulate(pairs, K, Mrows, N, seed=K + Mrows + N)
    assert np.array_equal(T, ref)


def test_emulator_fails_a_dropped_lds_wait(monkeypatch):
    monkeypatch.setattr(G.Emit, "need", lambda self, regs: None)
    with pytest.raises(E.Race):
        E.emulate(False, 768, 256, 128)


def test_emulator_fails_a_copy_wait_that_lets_the_next_group_in_flight(monkeypatch):
    monkeypatch.setattr(G, "DPG", 2 * G.DPG)
    with pytest.raises(E.Race):
        E.emulate(False, 768, 256, 128)


def test_emulator_fails_swapped_scales(monkeypatch):
    def bad(e):
        e.need({G.V_MP, G.V_MP + 1})
        e(f"v_and_b32 v{G.V_MX}, 0xffff, v{G.V_MP + 1}")
        e(f"v_lshrrev_b32 v{G.V_MX + 1}, 16, v{G.V_MP}")
        e(f"v_and_b32 v{G.V_MX + 2}, 0xffff, v{G.V_MP}")
        e(f"v_lshrrev_b32 v{G.V_MX + 3}, 16, v{G.V_MP + 1}")
    monkeypatch.setattr(G, "extract_scales", bad)
    T, ref = E.emulate(False, 768, 256, 128)
    assert not np.array_equal(T, ref)
