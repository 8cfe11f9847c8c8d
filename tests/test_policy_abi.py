"""Binary compatibility of TileGatingPolicy with the reference header.

A policy subclass compiled against the reference's own header
(src/tile_gating_policy.h:8-17, read in place under /root/reference, never
copied) is handed to code compiled against this repository's header, which
calls its virtual select() and name() and this library's non-virtual
select_range() on it. Matching virtual tables make every call land in the
subclass; a virtual member added to this header would shift the slots (the
test then calls the wrong function). Skipped where the reference tree is
absent (it exists only in the build container)."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_HDR_DIR = Path("/root/reference/src")
LIB_DIR = ROOT / "cuda-kv-persistence_amd" / "lib"

SUBCLASS = r"""
#include "tile_gating_policy.h"   // the reference header
// Picks the highest-scoring candidate ids, descending by score.
class TopScorePolicy : public TileGatingPolicy {
public:
    void select(const float* s, int n, int max_tiles, long* out, int* count) override {
        int c = 0;
        for (int k = 0; k < max_tiles && k < n; ++k) {
            int best = -1;
            for (int i = 0; i < n; ++i) {
                bool used = false;
                for (int j = 0; j < c; ++j) used |= out[j] == i;
                if (!used && (best < 0 || s[i] > s[best])) best = i;
            }
            out[c++] = best;
        }
        *count = c;
    }
    const char* name() const override { return "top_score"; }
};
extern "C" TileGatingPolicy* make_top_score() { return new TopScorePolicy(); }
"""

DRIVER = r"""
#include <cstdio>
#include <cstring>
#include "tile_gating_policy.h"   // this repository's header
extern "C" TileGatingPolicy* make_top_score();
int main() {
    TileGatingPolicy* p = make_top_score();
    const float s[8] = {0.1f, 0.9f, 0.3f, 0.8f, 0.2f, 0.7f, 0.0f, 0.6f};
    long ids[8];
    int n = 0;
    p->select(s, 8, 3, ids, &n);
    if (n != 3 || ids[0] != 1 || ids[1] != 3 || ids[2] != 5) return 1;
    if (std::strcmp(p->name(), "top_score") != 0) return 2;
    // candidates 4..7 only: scores 0.2 0.7 0.0 0.6 -> ids 5, 7 (absolute)
    p->select_range(s, 4, 4, 2, ids, &n);
    if (n != 2 || ids[0] != 5 || ids[1] != 7) return 3;
    delete p;  // virtual destructor slot
    std::printf("abi ok\n");
    return 0;
}
"""


@pytest.mark.skipif(not (REF_HDR_DIR / "tile_gating_policy.h").exists(),
                    reason="reference tree absent (build container only)")
@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ absent")
def test_reference_header_subclass_is_binary_compatible(tmp_path):
    (tmp_path / "sub.cpp").write_text(SUBCLASS)
    (tmp_path / "drv.cpp").write_text(DRIVER)
    subprocess.run(["g++", "-std=c++17", "-O1", "-fPIC", "-shared", f"-I{REF_HDR_DIR}",
                    "sub.cpp", "-o", "libsub.so"], cwd=tmp_path, check=True)
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{ROOT / 'include'}", "drv.cpp",
                    "-o", "drv", f"-L{tmp_path}", "-lsub", f"-L{LIB_DIR}", "-lkvpersist",
                    f"-Wl,-rpath,{tmp_path}:{LIB_DIR}"], cwd=tmp_path, check=True)
    r = subprocess.run([str(tmp_path / "drv")], capture_output=True, text=True)
    assert r.returncode == 0 and "abi ok" in r.stdout, (r.returncode, r.stdout, r.stderr)
