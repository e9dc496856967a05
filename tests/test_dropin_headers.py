"""CPU: the C++ drop-in's headers against the reference's own headers, read
from /root/reference when it is present (skipped elsewhere).

In the drop-in's include order (tiny-llm_amd/include first, then the
reference's include/), the library's directory may only stand in for the
headers it replaces in full -- tiny_llm/kv_cache.h, result.h and types.h --
and must leave every other tiny_llm/*.h, logger.h included, to the
reference.  types.h must declare every type of the reference's
include/tiny_llm/types.h with the same members, member types and defaults
(the fp16 type aside), so transformer.h, validator.h and inference_engine.h
keep compiling."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
OURS = os.path.join(ROOT, "tiny-llm_amd", "include")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "include", "tiny_llm")),
                                reason="reference tree not present")


def resolved_headers(tmp_path, includes):
    src = tmp_path / "deps.cpp"
    src.write_text("".join(f'#include "{h}"\n' for h in includes))
    r = subprocess.run([HIPCC, "-x", "c++", "-std=c++17", "-M", "-MG", "-I", OURS,
                        "-I", os.path.join(REF, "include"), "-I", os.path.join(REF, "kernels"),
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return [p for p in r.stdout.replace("\\\n", " ").split() if "tiny_llm/" in p]


def test_only_replaced_headers_resolve_to_the_library(tmp_path):
    deps = resolved_headers(tmp_path, ["tiny_llm/inference_engine.h", "tiny_llm/transformer.h",
                                       "tiny_llm/validator.h", "tiny_llm/logger.h",
                                       "tiny_llm/kv_cache.h"])
    ours = {os.path.basename(p) for p in deps if os.path.realpath(p).startswith(OURS)}
    theirs = {os.path.basename(p) for p in deps if os.path.realpath(p).startswith(REF)}
    assert ours == {"kv_cache.h", "result.h", "types.h", "hip_utils.h"}, ours
    assert {"logger.h", "transformer.h", "validator.h", "inference_engine.h"} <= theirs, theirs
    assert not os.path.exists(os.path.join(OURS, "tiny_llm", "logger.h"))


def test_reference_validator_compiles_against_the_library_headers(tmp_path):
    src = tmp_path / "tu.cpp"
    src.write_text('#include "tiny_llm/kv_cache.h"\n#include "tiny_llm/validator.h"\n'
                   "int use(const tiny_llm::ModelConfig &m, const tiny_llm::GenerationConfig &g,\n"
                   "        const tiny_llm::KVCacheConfig &k) {\n"
                   "  return m.num_kv_heads + g.top_k + k.max_batch_size;\n}\n")
    r = subprocess.run([HIPCC, "-std=c++17", "-fsyntax-only", "-I", OURS,
                        "-I", os.path.join(REF, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def reference_struct_members():
    """(struct, member, type text, default text or None) of every data
    member of the reference's types.h."""
    text = open(os.path.join(REF, "include", "tiny_llm", "types.h")).read()
    text = re.sub(r"//[^\n]*", "", text)
    out = []
    for m in re.finditer(r"struct\s+(\w+)\s*\{(.*?)\n\};", text, flags=re.S):
        name, body = m.group(1), m.group(2)
        depth = 0
        for line in body.splitlines():
            s = line.strip()
            if depth == 0 and s.endswith(";") and "(" not in s:
                decl = s[:-1]
                default = None
                if "=" in decl:
                    decl, default = (x.strip() for x in decl.split("=", 1))
                mm = re.match(r"(.+?)\s*(\w+)$", decl)
                out.append((name, mm.group(2), mm.group(1).strip(), default))
            depth += s.count("{") - s.count("}")
    return out


def test_types_header_matches_the_reference(tmp_path):
    members = reference_struct_members()
    assert len(members) > 40
    checks = []
    for struct, member, typ, default in members:
        checks.append(f"static_assert(std::is_same_v<decltype({struct}::{member}), {typ}>, "
                      f'"{struct}::{member}");')
        if default is not None:
            checks.append(f"if (!({struct}{{}}.{member} == {default})) "
                          f'{{ std::puts("default {struct}::{member}"); return 1; }}')
    src = tmp_path / "members.cpp"
    src.write_text('#include "tiny_llm/types.h"\n#include <cstdio>\n#include <type_traits>\n'
                   "namespace tiny_llm {\nint check() {\n" + "\n".join(checks) +
                   "\nreturn 0;\n}\n}\nint main() { return tiny_llm::check(); }\n")
    exe = tmp_path / "members"
    r = subprocess.run([HIPCC, "-std=c++17", "-I", OURS, str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout
