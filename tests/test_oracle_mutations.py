"""The pins in test_oracle_traces.py are strong enough to catch plausible
mistakes in the oracle's controller and loop sequencing: each mutation below
is planted in a temporary copy of oracle/fg_oracle.c (compiled on the CPU,
loaded through FG_ORACLE_LIB in a separate pytest process), and the pin tests
must fail against it.  The unmutated copy must pass them."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "fg_oracle.c")

MUTATIONS = {
    "stall threshold 4 -> 3": ("stall >= 4", "stall >= 3"),
    "first instead of last expander distance": (
        "st->current_expander_distance = parent_dist[n_parents - 1];",
        "st->current_expander_distance = parent_dist[0];"),
    "rho span rho2 - 0.25 -> rho2": (
        "phase2_rho > 0.25f ? phase2_rho - 0.25f : 0.99f - 0.0f",
        "phase2_rho > 0.25f ? phase2_rho : 0.99f - 0.0f"),
    "K-th cutoff one slot early": (
        "return beam_dist[(K < beam ? K : beam) - 1];",
        "return beam_dist[(K < beam ? K : beam) > 1 ? (K < beam ? K : beam) - 2 : 0];"),
    "stage-I near count <= -> <": ("cd[i] <= kth_cutoff);", "cd[i] < kth_cutoff);"),
    "stage-II near count <= -> <": ("est[l] <= kth_cutoff);", "est[l] < kth_cutoff);"),
    "visited reset every 15 iterations": (
        "(iter + 1) % FGO_HASH_RESET == 0", "(iter + 1) % (FGO_HASH_RESET - 1) == 0"),
    "max_iter = beam": ("const int max_iter = (beam_sz * 11 + 9) / 10;", "const int max_iter = beam_sz;"),
    "stage-II keep + 1": (
        "eff = fgo_keep_count_for_expander(an, st.spec_degree, st.rho, kth_valid, near);",
        "eff = fgo_keep_count_for_expander(an, st.spec_degree, st.rho, kth_valid, near) + 1;"),
    "no final merge after the loop": (
        "fgo_merge_candidates(bd, bi, cd, ci, cbs, pbeam, 0, ws->scratch_d, ws->scratch_i);  /* :449-451 */",
        "/* final merge dropped */"),
}


def _build(tmp_path, name, mutation):
    src = open(SRC).read()
    if mutation is not None:
        old, new = mutation
        assert src.count(old) == 1, f"mutation site not unique: {old}"
        src = src.replace(old, new)
    d = tmp_path / name
    d.mkdir()
    (d / "fg_oracle.c").write_text(src)
    so = d / "liboracle.so"
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-pthread",
                    "-I", os.path.join(ROOT, "oracle"), "-o", str(so), str(d / "fg_oracle.c"), "-lm"], check=True)
    return str(so)


def _pins_pass(lib):
    env = dict(os.environ, FG_ORACLE_LIB=lib)
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_oracle_traces.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    return r.returncode == 0, r.stdout[-400:]


def test_unmutated_copy_passes(tmp_path):
    ok, out = _pins_pass(_build(tmp_path, "clean", None))
    assert ok, out


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_mutation_is_caught(tmp_path, name):
    ok, out = _pins_pass(_build(tmp_path, "m", MUTATIONS[name]))
    assert not ok, f"the pin tests pass with the mutation '{name}' planted"
