"""The reference-harness patch in INTEGRATION.md compiles and links.

The file-scope block and the one-line changes are taken from INTEGRATION.md
as they stand and compiled with g++ against gat-tfs_amd/host/gat_types.hpp,
whose containers carry the field names of baseline/include/gat.hpp:32-106
(the reference's own header needs oneMKL, absent here), then linked against
libgatgpu.so.  No GPU is touched: the program only checks the path names.
"""
import re
import subprocess
from pathlib import Path

import gatgpu

ROOT = Path(__file__).resolve().parent.parent


def patch_pieces():
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```cpp\n(.*?)```", text, re.S)
    scope = next(b for b in blocks if "// integration: file scope" in b)
    change1 = next(b.strip() for b in blocks if b.strip().startswith("if(gpu_run_path("))
    change3 = next(b.strip() for b in blocks if b.strip() == "g_model=&model;")
    change5 = next(b for b in blocks if "gpu_model_seconds(path" in b and "double total;" in b)
    gpu_branch = change5.split("else")[0]  # the GPU branch of the benchmark timer
    return scope, change1, change3, gpu_branch


def test_integration_patch_compiles_and_links(tmp_path):
    gatgpu.load_library()  # built
    scope, change1, change3, gpu_branch = patch_pieces()
    src = f"""
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>
#include "gat_types.hpp"
using namespace gat;
{scope}
static void run_path(const std::string& path, const Graph& g, const Param& p, const std::vector<float>& input,
                     Workspace& w, bool hidden, Times& t) {{
    {change1}
    throw std::runtime_error("bad path");
}}
static double bench_once(const std::string& path, const Graph& g, const Model& model, int layer) {{
    Workspace ws[3];
    Times times[3];
    const std::vector<float>* input = &g.x;
    {gpu_branch}
    (void)input;
    return total;
}}
int main(int argc, char**) {{
    Model model(3);
    Graph g;
    {change3}
    if (argc > 99) {{  // compiled and linked, never run here
        Workspace w;
        Times t;
        run_path("gpu_bf16", g, model[0], g.x, w, true, t);
        std::printf("%f\\n", bench_once("gpu_fp32", g, model, 0));
    }}
    return is_gpu_path("gpu_bf16") && is_gpu_path("gpu_fp32") && !is_gpu_path("standard_bf16") ? 0 : 1;
}}
"""
    f = tmp_path / "patch.cpp"
    f.write_text(src)
    lib = ROOT / "gat-tfs_amd" / "lib"
    exe = tmp_path / "patch"
    p = subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-Wno-unused-function", f"-I{ROOT / 'include'}",
                        f"-I{ROOT / 'gat-tfs_amd' / 'host'}", str(f), str(ROOT / "gat-tfs_amd" / "host" / "gat_types.cpp"),
                        f"-L{lib}", "-lgatgpu", f"-Wl,-rpath,{lib}", "-o", str(exe)],
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stderr[-3000:]
    assert subprocess.run([str(exe)], timeout=60).returncode == 0
