"""Host regression test of the buffer-descriptor address recombination
(gpt_amd/csrc/attn_addr.h, used by make_rsrc in attn_common.h).

Every head_dim-64 kernel builds its buffer descriptors from a base address
whose two 32-bit words are broadcast with readfirstlane (int -> int). If the
low word is widened through int, every address with bit 31 set comes back
with its high word replaced by 0xffffffff, and the kernels then address
memory they do not own. tests/addr_check.cpp compiles the header's function
with g++ and checks the round trip for such addresses; a copy of the function
that sign-extends the low word must fail the same check (the check can tell
the two apart)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _build_and_run(tmp_path, src_text=None):
    src = os.path.join(HERE, "addr_check.cpp")
    if src_text is not None:
        src = str(tmp_path / "addr_check_planted.cpp")
        with open(src, "w") as fh:
            fh.write(src_text)
    exe = str(tmp_path / "addr_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", HERE, src, "-o", exe], check=True)
    return subprocess.run([exe], capture_output=True, text=True)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_join_words_round_trip(tmp_path):
    r = _build_and_run(tmp_path)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok") and " with bit 31 set" in r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_sign_extending_join_is_caught(tmp_path):
    """The same check against a planted sign-extending recombination (a copy
    of the test program with its own join, not the product header)."""
    text = open(os.path.join(HERE, "addr_check.cpp")).read()
    planted = text.replace('#include "../gpt_amd/csrc/attn_addr.h"',
                           "#include <stdint.h>\nnamespace gpt_attn {\n"
                           "inline uint64_t join_words(int hi, int lo)\n"
                           "{ return ((uint64_t)(uint32_t)hi << 32) | (uint64_t)(int64_t)lo; }\n}")
    assert planted != text
    r = _build_and_run(tmp_path, planted)
    assert r.returncode == 1 and "FAIL:" in r.stdout and "mismatch: 00000000800" in r.stdout, r.stdout
