"""The int4-mode layout parse and its checks (load_int4, qwen_infer.c:554-615) through
bgl_int4_layout_check: no device work, so these run without a GPU.  Each refusal mirrors one FATAL
of the reference loader; parsing stops quietly at the first line without the seven leading fields,
as the reference's fscanf loop does."""
import os

import pytest

from loader_fixture import build


@pytest.fixture()
def model(oracle, tmp_path):
    return build(oracle, str(tmp_path))


def check(layout, blob):
    import beglin_amd
    return beglin_amd.layout_check(layout, blob)


def rewrite(layout, edit):
    lines = open(layout).read().splitlines()
    lines = edit(lines)
    with open(layout, "w") as f:
        f.write("\n".join(lines) + "\n")


def test_valid_layout(model):
    layout, blob, refs = model
    assert check(layout, blob) == (0, len(refs))


@pytest.mark.parametrize("case", [
    "misaligned_q4", "misaligned_g256", "missing_soff2", "g256_in", "g256_ng", "q4_in", "q4_ng", "q8_ng", "extent_q4",
    "extent_q8", "extent_g256_sub", "extent_f32", "unknown_kind", "duplicate", "negative_dim", "negative_off",
])
def test_refusals(model, case):
    layout, blob, _ = model
    wb = os.path.getsize(blob)

    def field(i, j, v):
        def ed(lines):
            f = lines[i].split()
            f[j] = str(v)
            lines[i] = " ".join(f)
            return lines
        return ed

    edits = {
        "misaligned_q4": field(0, 2, 8), "misaligned_g256": field(2, 7, int(open(layout).read().splitlines()[2].split()[7]) + 4),
        "missing_soff2": lambda L: L[:2] + [" ".join(L[2].split()[:7])],
        "g256_in": field(2, 4, 1024 + 64), "g256_ng": field(2, 5, 16), "q4_in": field(0, 4, 500), "q4_ng": field(0, 5, 9),
        "q8_ng": field(1, 5, 3), "extent_q4": field(0, 3, 100000), "extent_q8": field(1, 2, wb - 64),
        "extent_g256_sub": field(2, 7, wb - 64), "extent_f32": field(3, 3, wb),
        "unknown_kind": field(1, 1, "q6k"), "duplicate": field(1, 0, "q.proj"), "negative_dim": field(0, 3, -1),
        "negative_off": field(0, 2, -64),
    }
    rewrite(layout, edits[case])
    rc, _ = check(layout, blob)
    assert rc < 0, case


def test_too_many_tensors(oracle, tmp_path):
    layout, blob, _ = build(oracle, str(tmp_path), [("n", "f32", 4, 0)])
    with open(layout, "w") as f:
        f.write("".join(f"t{i} f32 0 4 0 0 0\n" for i in range(513)))
    assert check(layout, blob)[0] < 0
    with open(layout, "w") as f:
        f.write("".join(f"t{i} f32 0 4 0 0 0\n" for i in range(512)))
    assert check(layout, blob) == (0, 512)


def test_parse_stops_at_a_short_line(model):
    layout, blob, refs = model
    rewrite(layout, lambda L: L[:2] + ["garbage line"] + L[2:])
    assert check(layout, blob) == (0, 2)


def test_missing_files(model, tmp_path):
    layout, blob, _ = model
    assert check(str(tmp_path / "nope.txt"), blob)[0] < 0
    assert check(layout, str(tmp_path / "nope.bin"))[0] < 0


# ---------------------------------------------------------------- the AF layout manifest
def af_check(layout, blob):
    import beglin_amd
    return beglin_amd.af_layout_check(layout, blob.nbytes)


def test_af_valid_layout(tmp_path):
    from loader_fixture import build_af
    layout, blob, recs = build_af(str(tmp_path))
    assert af_check(layout, blob) == (0, len(recs))


@pytest.mark.parametrize("case", ["ng", "in64", "E0", "out0", "pb_short", "po_past", "so_past", "bo_past", "neg_off",
                                  "duplicate", "long_name", "huge"])
def test_af_refusals(tmp_path, case):
    from loader_fixture import build_af
    layout, blob, _ = build_af(str(tmp_path))
    wb = blob.nbytes

    def field(i, j, v):
        def ed(lines):
            f = lines[i].split()
            f[j] = str(v)
            lines[i] = " ".join(f)
            return lines
        return ed

    edits = {
        "ng": field(0, 4, 3), "in64": lambda L: field(0, 3, 96)(field(0, 4, 1)(L)), "E0": field(1, 1, 0),
        "out0": field(1, 2, 0), "pb_short": field(2, 6, 4 * 128 * 64 // 2 - 1), "po_past": field(3, 5, wb - 64),
        "so_past": field(3, 7, wb - 64), "bo_past": field(3, 8, wb), "neg_off": field(0, 7, -64),
        "duplicate": field(2, 0, "lm_head"), "long_name": field(1, 0, "x" * 128),
        # E * out * in past 64 bits: refused before any size is formed from it
        "huge": lambda L: field(0, 1, 2**31 - 1)(field(0, 2, 2**31 - 1)(field(0, 3, 2**31 - 64)(field(0, 4, (2**31 - 64) // 64)(L)))),
    }
    rewrite(layout, edits[case])
    rc, _ = af_check(layout, blob)
    assert rc < 0, case


def test_af_limits_and_short_records(tmp_path):
    from loader_fixture import build_af
    layout, blob, recs = build_af(str(tmp_path))
    rewrite(layout, lambda L: L[:2] + ["truncated 4 64"] + L[2:])       # the manifest ends at a short record
    assert af_check(layout, blob) == (0, 2)
    rec = open(layout).read().splitlines()[0].split()
    for n, want in ((1024, (0, 1024)), (1025, None)):
        with open(layout, "w") as f:
            f.write("".join(" ".join([f"t{i}"] + rec[1:]) + "\n" for i in range(n)))
        rc, cnt = af_check(layout, blob)
        assert (rc, cnt) == want if want else rc < 0
    assert af_check(str(tmp_path / "missing.txt"), blob)[0] < 0
