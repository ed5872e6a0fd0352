"""Build step: the reference engine's source with six static functions
replaced by the layer-level GPU versions in include/midge_hip_layer.inc.

    python oracle/mk_layer_engine.py <midge checkout>/engine/midge.c _ref/midge_layer.c

Each function is found by the first line of its definition and ends at the
next line that is a lone "}" (the reference's style for top-level
functions); its lines are replaced by an include of that function's part
of midge_hip_layer.inc. Everything else is the checkout's text, unchanged.
The output goes to oracle/_ref/ (git-ignored) and is compiled there; the
reference's source is never kept in this repository.
"""
import sys

# (first line of the definition, the part of midge_hip_layer.inc replacing it)
FUNCS = [
    ("static void preload_hot(Model *m, double gb) {", 1),
    ("static void moe(Model *m, int layer) {", 2),
    ("static void forward_batch(Model *m, const int *toks, int n, int tfall,", 3),
    ("static void forward(Model *m, int token, int want_logits) {", 4),
    ("static int sample(Model *m, float temp, float topp) {", 5),
    ("static void print_logits(Model *m) {", 6),
]


def transform(src: str) -> str:
    lines = src.split("\n")
    out, i, done = [], 0, set()
    while i < len(lines):
        hit = [part for sig, part in FUNCS if lines[i].startswith(sig)]
        if not hit:
            out.append(lines[i])
            i += 1
            continue
        j = i + 1
        while j < len(lines) and lines[j] != "}":
            j += 1
        if j == len(lines):
            raise SystemExit(f"no end for the function at line {i + 1}")
        part = hit[0]
        out += [f"#undef MH_LAYER_PART", f"#define MH_LAYER_PART {part}", '#include "midge_hip_layer.inc"']
        done.add(part)
        i = j + 1
    missing = {p for _, p in FUNCS} - done
    if missing:
        raise SystemExit(f"functions not found for parts {sorted(missing)}")
    return "\n".join(out)


if __name__ == "__main__":
    src, dst = sys.argv[1], sys.argv[2]
    with open(src) as f:
        text = transform(f.read())
    with open(dst, "w") as f:
        f.write(text)
