"""The oracle and the .qora-tts reader under AddressSanitizer and
UndefinedBehaviorSanitizer, on the CPU.  tests/sanitize.mk builds both with
every report fatal (gcc / g++; nothing for the GPU):

- the reader (csrc/model_file.cpp) runs a fuzz pass (tests/fuzz_model_file.cpp):
  truncations, rewritten counts and header fields, flipped bytes of a
  well-formed file; every accepted mutant is read back at the lengths the
  upload functions read, every rejected one must carry a message;
- the oracle's CPU tests run against the sanitized oracle build, with the
  sanitizer runtimes preloaded into the Python process.

A sanitizer report fails the test with the report in its output."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OUT = os.path.join(ROOT, "tests", "_build")


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.fixture(scope="module")
def built():
    if not (_runtime("libasan.so") and _runtime("libubsan.so")):
        pytest.skip("gcc has no AddressSanitizer / UndefinedBehaviorSanitizer runtime here")
    subprocess.run(["make", "-s", "-f", os.path.join("tests", "sanitize.mk")], cwd=ROOT, check=True)
    return OUT


@pytest.mark.timeout(600)
def test_reader_fuzz_pass(built, tmp_path):
    import qtts
    from oracle import oracle
    from qtts_file_writer import TextWeights, write_model
    from shapes import TINY_PREDICTOR, TINY_TALKER

    tw = qtts.TalkerWeights(41, TINY_TALKER)
    pw = qtts.CodePredictorWeights(41, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    text = TextWeights(41, text_vocab=96, text_hidden=64, hidden=TINY_TALKER.hidden)
    trope = oracle.build_rope_table(TINY_TALKER.head_dim, 64, TINY_TALKER.rope_theta)
    prope = oracle.build_rope_table(TINY_PREDICTOR.head_dim, 32, TINY_PREDICTOR.rope_theta)
    seed_file = str(tmp_path / "seed.qora-tts")
    write_model(seed_file, tw, pw, text, trope, prope)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    r = subprocess.run([os.path.join(built, "fuzz_model_file"), seed_file, "1500", "7", str(tmp_path / "mutant")],
                       capture_output=True, text=True, env=env, timeout=500)
    print(r.stdout)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "1500 mutants" in r.stdout


@pytest.mark.timeout(900)
def test_oracle_suite_under_sanitizers(built):
    lib = os.path.join(built, "liboracle_asan.so")
    env = dict(os.environ, LD_PRELOAD=f"{_runtime('libasan.so')}:{_runtime('libubsan.so')}",
               ASAN_OPTIONS="detect_leaks=0", QTTS_ORACLE_LIB=lib)
    # the sanitized build is the one the oracle binding loads
    probe = ("import sys; sys.path[:0] = ['tests', 'qora-tts-12hz-1.7b_amd', '.']; from oracle import oracle; "
             "oracle.load(); maps = open('/proc/self/maps').read(); "
             "assert 'liboracle_asan.so' in maps and '/liboracle.so' not in maps, 'wrong oracle build'")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-4000:]
    tests = ["tests/test_oracle.py", "tests/test_oracle_decoder.py", "tests/test_oracle_legacy.py",
             "tests/test_oracle_prompt.py"]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu", *tests],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=840)
    print(r.stdout[-2000:])
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
