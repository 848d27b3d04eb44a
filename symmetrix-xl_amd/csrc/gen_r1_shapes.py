"""Generates r1_shapes.inc: compile-time path lists and CG sparsity patterns.

The second-interaction kernels unroll their term loops over these patterns so
that per-receiver accumulators stay in registers.  The coefficient values are
not compiled in: the evaluator reads them from the model JSON at load time
(``Phi1_clebsch_gordan``) and rejects a model whose terms fall outside the
compiled pattern of its (l_max, L_max).

Run from the repository root:  python symmetrix-xl_amd/csrc/gen_r1_shapes.py
"""

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from symmetrix_amd import irreps  # noqa: E402

SHAPES = [(2, 1), (3, 1), (3, 2), (3, 0), (2, 0), (2, 2)]
# Shapes whose per-channel reverse state does not fit the register file in
# one pass run the second-interaction reverse in passes over disjoint path
# groups by source l2: each pass owns its message rows and edge forces add up
# over passes.  (Forward passes by output l were measured slower on the wide
# shape than one pass: every extra sweep re-reads the source features.)  The
# wide shape runs two passes, source l2 in {0, 1} and {2}, at two waves per
# SIMD; one pass spills, three repeat more per-edge work.  Passes only pay where one pass does not fit: the medium shape split
# in two (164 VGPRs, three waves per SIMD) was measured 33 % slower.
REV_GROUPS = {(3, 2): [[0, 1], [2]]}
# A pass holds its CG-contracted dPhi1 per (path, lm2, lm1) triple in
# registers ("factored": two FMAs per triple and edge, no coefficient
# operand) up to this many triples; the wide shape's passes hold 76 and 111
# (241 VGPRs, no spills).  Beyond it a pass contracts per term with dPhi1 rows
# in registers.
FACTORED_MAX_TRIPLES = 128


def emit_shape(lmax, Lmax):
    t = irreps.phi1_tables(lmax, Lmax)
    paths = t["paths"]
    num_e = t["num_e"]
    path_e, counts = [], [0] * (lmax + 1)
    for _, _, lo in paths:
        path_e.append(counts[lo])
        counts[lo] += 1
    lme_off, off = [], 0
    for l in range(lmax + 1):
        lme_off.append(off)
        off += (2 * l + 1) * num_e[l]
    nlme = off
    row0, r = [], 0
    for l1, l2, _ in paths:
        row0.append(r)
        r += (2 * l1 + 1) * (2 * l2 + 1)
    nrows = r
    row_path = []
    for p, (l1, l2, _) in enumerate(paths):
        row_path += [p] * ((2 * l1 + 1) * (2 * l2 + 1))
    terms = []
    for term in t["terms"]:
        p = row_path[term["row"]]
        terms.append((p, term["lm2"], term["lm1"], term["lme"], term["row"]))
    terms.sort()
    # (path, lm2) pairs and (path, lm2, lm1) triples in term order
    pqs, triples, term_tr = [], [], []
    for p, lm2, lm1, _, _ in terms:
        if (p, lm2) not in pqs:
            pqs.append((p, lm2))
        if (p, lm2, lm1) not in triples:
            triples.append((p, lm2, lm1))
        term_tr.append(triples.index((p, lm2, lm1)))
    # distinct (path, lm2, lme) groups in term order: the forward pass folds
    # the terms of a group into one per-edge weight sum_t cg_t Y[lm1_t]
    pls, term_pl = [], []
    for p, lm2, _, lme, _ in terms:
        if (p, lm2, lme) not in pls:
            pls.append((p, lm2, lme))
        term_pl.append(pls.index((p, lm2, lme)))
    name = f"R1Shape<{lmax}, {Lmax}>"

    def arr(vals):
        return "{" + ", ".join(str(v) for v in vals) + "}"

    groups = emit_groups(lmax, Lmax, paths, terms)

    lines = [
        "template <>",
        f"struct {name} {{",
        f"    static constexpr int LMAX = {lmax};",
        f"    static constexpr int LLMAX = {Lmax};",
        f"    static constexpr int NP = {len(paths)};",
        f"    static constexpr int NT = {len(terms)};",
        f"    static constexpr int NLME = {nlme};",
        f"    static constexpr int NROWS = {nrows};",
        f"    static constexpr int path_l1[NP] = {arr([p[0] for p in paths])};",
        f"    static constexpr int path_l2[NP] = {arr([p[1] for p in paths])};",
        f"    static constexpr int path_lo[NP] = {arr([p[2] for p in paths])};",
        f"    static constexpr int path_e[NP] = {arr(path_e)};",
        f"    static constexpr int path_row0[NP] = {arr(row0)};",
        f"    static constexpr int num_e[LMAX + 1] = {arr(num_e)};",
        f"    static constexpr int lme_off[LMAX + 1] = {arr(lme_off)};",
        "    // terms sorted by (path, lm2, lm1, lme)",
        f"    static constexpr int term_p[NT] = {arr([x[0] for x in terms])};",
        f"    static constexpr int term_lm2[NT] = {arr([x[1] for x in terms])};",
        f"    static constexpr int term_lm1[NT] = {arr([x[2] for x in terms])};",
        f"    static constexpr int term_lme[NT] = {arr([x[3] for x in terms])};",
        f"    static constexpr int term_row[NT] = {arr([x[4] for x in terms])};",
        "    // distinct (path, lm2) pairs and (path, lm2, lm1) triples, term order",
        f"    static constexpr int NPQ = {len(pqs)};",
        f"    static constexpr int pq_p[NPQ] = {arr([x[0] for x in pqs])};",
        f"    static constexpr int pq_lm2[NPQ] = {arr([x[1] for x in pqs])};",
        f"    static constexpr int NTR = {len(triples)};",
        f"    static constexpr int tr_pq[NTR] = {arr([pqs.index(x[:2]) for x in triples])};",
        f"    static constexpr int tr_lm1[NTR] = {arr([x[2] for x in triples])};",
        f"    static constexpr int term_tr[NT] = {arr(term_tr)};",
        "    // distinct (path, lm2, lme) groups, term order",
        f"    static constexpr int NPL = {len(pls)};",
        f"    static constexpr int pl_pq[NPL] = {arr([pqs.index(x[:2]) for x in pls])};",
        f"    static constexpr int pl_lme[NPL] = {arr([x[2] for x in pls])};",
        f"    static constexpr int term_pl[NT] = {arr(term_pl)};",
        "};",
        "",
    ]
    return "\n".join(lines) + groups


def _arr(vals):
    return "{" + ", ".join(str(v) for v in vals) + "}"


def emit_groups(lmax, Lmax, paths, terms):
    """Pass structures of a grouped shape.  `terms` is the shape's sorted
    term list (path, lm2, lm1, lme, row); group arrays index it."""
    rev = REV_GROUPS.get((lmax, Lmax), [])
    if not rev:
        return ""
    out = [
        "template <>",
        f"struct R1Groups<{lmax}, {Lmax}> {{",
        f"    static constexpr int NREV = {len(rev)};",
        "};",
        "",
    ]
    for g, l2s in enumerate(rev):
        gp = [p for p, (_, l2, _) in enumerate(paths) if l2 in l2s]
        ts = [t for t, x in enumerate(terms) if x[0] in gp]
        rows = sorted({terms[t][3] for t in ts})
        pqs, trs = [], []
        for t in ts:
            p, lm2, lm1 = terms[t][:3]
            if (p, lm2) not in pqs:
                pqs.append((p, lm2))
            if (p, lm2, lm1) not in trs:
                trs.append((p, lm2, lm1))
        hl = sorted({lm2 for _, lm2 in pqs})
        factored = len(trs) <= FACTORED_MAX_TRIPLES
        out += [
            "template <>",
            f"struct R1RevGroup<{lmax}, {Lmax}, {g}> {{",
            f"    // source l2 in {l2s}",
            f"    static constexpr bool FACTORED = {'true' if factored else 'false'};",
            f"    static constexpr int NP = {len(gp)};",
            f"    static constexpr int path[NP] = {_arr(gp)};",
            f"    static constexpr int NH = {len(hl)};",
            f"    static constexpr int h_lm2[NH] = {_arr(hl)};",
            f"    static constexpr int NROW = {len(rows)};",
            f"    static constexpr int row_lme[NROW] = {_arr(rows)};",
            f"    static constexpr int NPQ = {len(pqs)};",
            f"    static constexpr int pq_p[NPQ] = {_arr([gp.index(p) for p, _ in pqs])};",
            f"    static constexpr int pq_h[NPQ] = {_arr([hl.index(lm2) for _, lm2 in pqs])};",
            f"    static constexpr int NTR = {len(trs)};",
            f"    static constexpr int tr_pq[NTR] = {_arr([pqs.index(x[:2]) for x in trs])};",
            f"    static constexpr int tr_lm1[NTR] = {_arr([x[2] for x in trs])};",
            f"    static constexpr int NT = {len(ts)};",
            f"    static constexpr int term[NT] = {_arr(ts)};",
            f"    static constexpr int term_lm1[NT] = {_arr([terms[t][2] for t in ts])};",
            f"    static constexpr int term_row[NT] = {_arr([rows.index(terms[t][3]) for t in ts])};",
            f"    static constexpr int term_tr[NT] = {_arr([trs.index(terms[t][:3]) for t in ts])};",
            "};",
            "",
        ]
    return "\n".join(out)


def render():
    """The text of r1_shapes.inc."""
    out = [
        "// Generated by gen_r1_shapes.py -- do not edit.",
        "// Path lists and CG sparsity of the second interaction for the",
        "// compiled (l_max, L_max) shapes; values come from the model JSON.",
        "#pragma once",
        "",
        "template <int LMAX, int LLMAX>",
        "struct R1Shape;",
        "",
        "// reverse pass structure of the shapes run in path-group passes (none: one pass)",
        "template <int LMAX, int LLMAX>",
        "struct R1Groups {",
        "    static constexpr int NREV = 0;",
        "};",
        "template <int LMAX, int LLMAX, int G>",
        "struct R1RevGroup;",
        "",
    ]
    for lmax, Lmax in SHAPES:
        out.append(emit_shape(lmax, Lmax))
    return "\n".join(out)


def main():
    path = os.path.join(HERE, "r1_shapes.inc")
    with open(path, "w") as f:
        f.write(render())
    print(path)


if __name__ == "__main__":
    main()
