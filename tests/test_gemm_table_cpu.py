"""The shipped GEMM solution table parses and names its library versions."""
from __future__ import annotations


def test_table_names_versions_and_shapes():
    from thetascan_amd import gemm_solutions

    validators, entries = gemm_solutions.read_table()
    assert validators["GCN_ARCH_NAME"].startswith("gfx950")
    for key in ("PT_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION"):
        assert validators[key]
    assert entries
    for op, problem, solution, ms in entries:
        assert op.startswith("GemmTunableOp_BFloat16_")
        assert solution.startswith(("Gemm_Hipblaslt_", "Gemm_Rocblas_"))
        assert ms > 0
    # the three projection shapes of a B8 x T4096, d_model 512 step
    problems = {p.split("_ld_")[0] for _, p, _, _ in entries}
    assert {"tn_2048_32768_512", "tn_512_32768_512", "nn_512_32768_512"} <= problems
