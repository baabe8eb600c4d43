"""The oracle's pins are strong enough to catch plausible mistakes in its
controller, loop sequencing, merge, stage-II selection, task order, id
validity, distance reduction, result writer, entry point and recall:
each mutation below is planted in a temporary copy of oracle/fg_oracle.c
(compiled on the CPU, loaded through FG_ORACLE_LIB in a separate pytest
process), and the pin tests (hand-traced searches, hand-computed primitives
and the merge-path tie case) must fail against it.  The unmutated copy must
pass them."""
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
    "merge-path ties go to the candidate": (
        "beam_d[ti] <= cand_d[ci]", "beam_d[ti] < cand_d[ci]"),
    "result writer tests MAX_INDEX before masking": (
        """        const uint32_t r = i < beam_sz ? (bi[i] & 0x7fffffffu) : FGO_MAX_INDEX;
        if (r != FGO_MAX_INDEX) last = r;
        out[i] = r == FGO_MAX_INDEX ? last : r;""",
        """        const uint32_t r = i < beam_sz ? bi[i] : FGO_MAX_INDEX;
        if (r != FGO_MAX_INDEX) last = r & 0x7fffffffu;
        out[i] = r == FGO_MAX_INDEX ? last : (r & 0x7fffffffu);"""),
    "stage-II estimates from the first parent's distance": (
        "fvq[l], pdist[pidx], B);", "fvq[l], pdist[0], B);"),
    "stage-II rank ties go to the higher lane": (
        "(other == mine && s < l)", "(other == mine && s > l)"),
    "stage-II keep-all >= -> >": (
        "const int keep_all = keep >= (int)raw_valid;", "const int keep_all = keep > (int)raw_valid;"),
    "stage-I keep-all >= -> >": (
        "const int keep_all = keep >= (int)valid;", "const int keep_all = keep > (int)valid;"),
    "partial tile counted as a full one": (
        "uint32_t an = active ? deg - (uint32_t)tile * 32u : 0u;",
        "uint32_t an = active ? (deg < 32u ? deg : 32u) : 0u;"),
    "no final merge after the loop": (
        "fgo_merge_candidates(bd, bi, cd, ci, cbs, pbeam, 0, ws->scratch_d, ws->scratch_i);  /* :449-451 */",
        "/* final merge dropped */"),
    "per-parent budget rounded up": (
        "(uint32_t)FGO_BUFFER_BOUND / (uint32_t)theta;",
        "((uint32_t)FGO_BUFFER_BOUND + (uint32_t)theta - 1) / (uint32_t)theta;"),
    "merge-path threads not rounded to a multiple of 32": ("    active = ((active + 31) / 32) * 32;\n", ""),
    "stage-I rate capped at RHO_MAX instead of the phase-2 rate": (
        "const float cap = phase2_rho > 0.25f ? phase2_rho : 0.99f;", "const float cap = 0.99f;"),
    "unfinite current expander falls back to the entry": (
        "*cur = finite_below_max(prev->current_expander_distance) ? prev->current_expander_distance : *last;",
        "*cur = finite_below_max(prev->current_expander_distance) ? prev->current_expander_distance : entry;"),
    "record falls back to the last distance": (
        "? st->current_expander_distance : st->entry_distance;",
        "? st->current_expander_distance : st->last_expander_distance;"),
    "stage-II tasks tile by tile": (
        """const uint32_t pidx = active ? (uint32_t)(task / tiles) : 0u;
                    const int tile = active ? task - (int)pidx * tiles : 0;""",
        """const uint32_t pidx = active ? (uint32_t)(task % (int)nexp) : 0u;
                    const int tile = active ? task / (int)nexp : 0;"""),
    "distance lanes summed in order instead of the shfl_down tree": (
        """    for (int off = 16; off >= 1; off >>= 1)
        for (int l = 0; l < off; ++l) v[l] = v[l] + v[l + off];
    return v[0];
}

/* utils.cuh:286-300 */""",
        """    for (int l = 1; l < 32; ++l) v[0] = v[0] + v[l];
    return v[0];
}

/* utils.cuh:286-300 */"""),
    "stage-I out-of-range ids valid": (
        "if (child >= ix->npoints || fgo_hash_contains(hash, bitlen, child)) child = FGO_MAX_INDEX;",
        "if (child == FGO_MAX_INDEX || fgo_hash_contains(hash, bitlen, child)) child = FGO_MAX_INDEX;"),
    "stage-II estimate from the tile's slot l instead of neighbour slot nidx": (
        "est[l] = fgo_estimate_seq(qf, codes + (size_t)nidx * bytes_per_nbr, tx[l], fdq[l],",
        "est[l] = fgo_estimate_seq(qf, codes + (size_t)l * bytes_per_nbr, tx[l], fdq[l],"),
    "query range over the d input dimensions only": (
        "    for (int i = 0; i < padded_dim; ++i) {\n        lo = fminf(lo, qf->rotated[i]);",
        "    for (int i = 0; i < dim; ++i) {\n        lo = fminf(lo, qf->rotated[i]);"),
    "entry point keeps the last of equal distances": (
        "        if (dd < best_dist) { best_dist = dd; best = (uint32_t)i; }",
        "        if (dd <= best_dist) { best_dist = dd; best = (uint32_t)i; }"),
    "entry-point centroid divides instead of scaling by fl(1/n)": (
        "            float t = row[d] * inv;", "            float t = row[d] / (float)npoints;"),
    "recall over all ground-truth columns": (
        "    const int eval_k = topk < gt_k ? topk : gt_k;", "    const int eval_k = gt_k;"),
    "recall counts a prediction once per matching column": (
        "                if (p == gt[i * (uint64_t)gt_k + k]) { ++correct; break; }",
        "                if (p == gt[i * (uint64_t)gt_k + k]) { ++correct; }"),
    "stage-II inserts of a round in reverse task order": (
        """                for (int w = 0; w < FGO_SEARCH_WIDTH; ++w)
                    for (int l = 0; l < 32; ++l) {
                        if (!keepl[w][l]) continue;""",
        """                for (int w = FGO_SEARCH_WIDTH - 1; w >= 0; --w)
                    for (int l = 0; l < 32; ++l) {
                        if (!keepl[w][l]) continue;"""),
    "stage-II tests see the round's earlier inserts": (
        """                    if (keep_all) {
                        for (int l = 0; l < 32; ++l) keepl[w][l] = valid[l];
                    } else {
                        fgo_warp_keep_topk(est, valid, eff, keepl[w]);
                    }
                }""",
        """                    if (keep_all) {
                        for (int l = 0; l < 32; ++l) keepl[w][l] = valid[l];
                    } else {
                        fgo_warp_keep_topk(est, valid, eff, keepl[w]);
                    }
                    for (int l = 0; l < 32; ++l) {
                        if (!keepl[w][l]) continue;
                        keepl[w][l] = 0;
                        if (!fgo_hash_insert(hash, bitlen, child[w][l])) continue;
                        const uint32_t slot = compact_count++;
                        if (slot < collect_cap) { ci[slot] = child[w][l]; cd[slot] = FLT_MAX; }
                    }
                }"""),
    "stage-II out-of-range ids valid": (
        "valid[l] = child[w][l] != FGO_MAX_INDEX && child[w][l] < ix->npoints &&",
        "valid[l] = child[w][l] != FGO_MAX_INDEX &&"),
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


PIN_TESTS = ["test_oracle_traces.py", "test_oracle_primitives.py",
             "test_oracle_networks.py::test_merge_path_ties_inside_segments_keep_beam_first",
             "test_oracle_networks.py::test_merge_path_segmentation_with_boundary_ties",
             "test_golden_ref_host.py"]


def _pins_pass(lib):
    env = dict(os.environ, FG_ORACLE_LIB=lib)
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider"] +
                       [os.path.join(ROOT, "tests", t) for t in PIN_TESTS],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    return r.returncode == 0, r.stdout[-400:]


def test_unmutated_copy_passes(tmp_path):
    ok, out = _pins_pass(_build(tmp_path, "clean", None))
    assert ok, out


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_mutation_is_caught(tmp_path, name):
    ok, out = _pins_pass(_build(tmp_path, "m", MUTATIONS[name]))
    assert not ok, f"the pin tests pass with the mutation '{name}' planted"
