"""The C ABI without a GPU: libgse.so loads, exports every function include/gse.h declares, reports its ABI version,
and the ctypes structs of goethe-engine_amd/_lib.py have the C layout (sizes and offsets read from a C program built
against the header with gcc)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gse.h")


def declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"GSE_API\s+[\w\s\*]+?\b(gse_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol(ge):
    names = declared()
    assert len(names) == 15, names
    L = C.CDLL(ge._lib.PATH)
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(ge._lib.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", ge._lib.PATH], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert {n for n in exported if n.startswith("gse_")} == set(names)


def test_abi_version(ge):
    L = ge._lib.bind()
    v = L.gse_abi_version()
    assert (v >> 16, v & 0xFFFF) == (ge._lib.ABI_MAJOR, ge._lib.ABI_MINOR)


PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "gse.h"
#define F(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  printf("gse_open_params %zu\n", sizeof(gse_open_params));
  printf("gse_row %zu\n", sizeof(gse_row));
  printf("gse_batch %zu\n", sizeof(gse_batch));
  printf("gse_out %zu\n", sizeof(gse_out));
  printf("gse_mss_batch %zu\n", sizeof(gse_mss_batch));
  printf("gse_qrows %zu\n", sizeof(gse_qrows));
  printf("gse_tree %zu\n", sizeof(gse_tree));
  printf("gse_tree_out %zu\n", sizeof(gse_tree_out));
  printf("gse_pick_batch %zu\n", sizeof(gse_pick_batch));
  %FIELDS%
  return 0;
}
"""


def test_struct_layouts_match_the_header(ge, tmp_path):
    lib = ge._lib
    pairs = [("gse_open_params", lib.OpenParams), ("gse_batch", lib.Batch), ("gse_out", lib.Out),
             ("gse_mss_batch", lib.MssBatch), ("gse_qrows", lib.QRows), ("gse_tree", lib.Tree),
             ("gse_tree_out", lib.TreeOut), ("gse_pick_batch", lib.PickBatch)]
    fields = []
    for cname, cls in pairs:
        for f, _ in cls._fields_:
            fields.append(f"F({cname}, {f})")
    for f in lib.ROW.names:
        fields.append(f"F(gse_row, {f})")
    src = tmp_path / "probe.c"
    src.write_text(PROBE.replace("%FIELDS%", "\n  ".join(fields)))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(ln.rsplit(" ", 1) for ln in subprocess.run([str(exe)], capture_output=True, text=True,
                                                            check=True).stdout.splitlines())
    for cname, cls in pairs:
        assert int(got[cname]) == C.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(cls, f).offset, (cname, f)
    assert int(got["gse_row"]) == lib.ROW.itemsize
    for f in lib.ROW.names:
        assert int(got[f"gse_row.{f}"]) == lib.ROW.fields[f][1], f


def test_row_record_round_trip(ge):
    r = np.zeros(2, dtype=ge._lib.ROW)
    r["temperature"] = [0.5, 0.0]
    r["top_p"] = [0.95, 1.0]
    r["seed"] = [2 ** 64 - 1, 7]
    raw = r.view(np.uint8)
    assert raw.shape == (2 * 72,)
    assert np.frombuffer(raw[:4].tobytes(), np.float32)[0] == np.float32(0.5)
    assert np.frombuffer(raw[40:48].tobytes(), np.uint64)[0] == 2 ** 64 - 1


ENUMS = r"""
#include <stdio.h>
#include "gse.h"
int main(void) {
  printf("%u %u %u %u\n", (unsigned)GSE_BATCH_EXACT, (unsigned)GSE_BATCH_PROFILE, (unsigned)GSE_BATCH_NO_PLAN_WAIT,
         (unsigned)GSE_BATCH_NO_SPLIT);
  return 0;
}
"""


def test_batch_flags_match_the_header(ge, tmp_path):
    """The GSE_BATCH_* bits the binding uses are the header's."""
    src = tmp_path / "enums.c"
    src.write_text(ENUMS)
    exe = tmp_path / "enums"
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    subprocess.run(["gcc", "-I", inc, str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    lib = ge._lib
    assert got == [lib.BATCH_EXACT, lib.BATCH_PROFILE, lib.BATCH_NO_PLAN_WAIT, lib.BATCH_NO_SPLIT]
