"""The forword.c side of the boundary as INTEGRATION.md section 1 writes it,
compiled against the reference's own headers (transformer.h:15-48,
gguf.h:16-39, model_config.h:47-95) with the reference's warning flags plus
-DFORWORD_GPU -Werror, and linked against libforword_gpu.so with every symbol
resolved.  CPU only: nothing is run.  Skipped where the reference sources are
absent (they never travel with the repository)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
LIB = os.path.join(ROOT, "forword.c_amd", "lib")

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(REF, "transformer.h")),
                                reason="reference headers not present")


def glue_blocks():
    """The C blocks of INTEGRATION.md section 1, in order."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 1."):text.index("## 2.")]
    return re.findall(r"```c\n(.*?)```", sec, re.S)


def patched_transformer_h(block):
    """The reference's transformer.h with the field block 1 adds: the include
    before the struct and `forword_gpu_t *gpu` as its last member."""
    src = open(os.path.join(REF, "transformer.h")).read()
    inc = block[block.index("#ifdef FORWORD_GPU"):block.index("#endif") + len("#endif")]
    field = re.search(r"(#ifdef FORWORD_GPU\s*\n\s*forword_gpu_t \*gpu;\s*\n#endif)", block).group(1)
    src = src.replace("typedef struct {", inc + "\ntypedef struct {", 1)
    return src.replace("} transformer_t;", field + "\n} transformer_t;", 1)


def test_glue_compiles_against_reference_headers(tmp_path):
    blocks = glue_blocks()
    assert len(blocks) == 6, "INTEGRATION.md section 1 should hold six C blocks"
    hdr, init, fwd, free_, prefill, generate = blocks
    (tmp_path / "transformer.h").write_text(patched_transformer_h(hdr))
    unit = "\n".join([
        '#include <stdio.h>', '#include <stdlib.h>', '#include <string.h>',
        '#include "transformer.h"',
        "int glue_init(transformer_t *t)", "{", init, "    return 0;", "}",
        "float *glue_forward(transformer_t *t, uint32_t token_id, size_t pos)", "{", fwd,
        "}",
        "void glue_free(transformer_t *t)", "{", free_, "}",
        "int glue_prefill(transformer_t *t, const uint32_t *prompt, size_t n_prompt)", "{", prefill,
        "    return logits[0] > 0.0f;", "}",
        "int glue_generate(transformer_t *t, const uint32_t *prompt_ids, size_t prompt_n, size_t max_tokens,",
        "                  float temperature, float top_p, float rep_pen, uint64_t rng_seed)", "{", generate,
        "    int first = (int)ids[0];", "    free(ids);", "    return first;", "}",
    ])
    (tmp_path / "glue.c").write_text(unit)
    cc = shutil.which("gcc") or "cc"
    cmd = [cc, "-O2", "-std=c11", "-Wall", "-Wextra", "-Wpedantic", "-Werror", "-DFORWORD_GPU",
           "-fPIC", "-shared", f"-I{tmp_path}", f"-I{REF}", f"-I{os.path.join(ROOT, 'include')}",
           str(tmp_path / "glue.c"), "-o", str(tmp_path / "libglue.so"), f"-L{LIB}", "-lforword_gpu",
           "-Wl,--no-undefined", "-Wl,-rpath-link,/opt/rocm/lib", f"-Wl,-rpath,{LIB}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
