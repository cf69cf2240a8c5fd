"""The safetensors reader (sltx_st_*) over the committed corpus of truncated,
mutated and hand-made headers (tests/golden/st_corpus, written by
tests/golden/make_st_corpus.py).  Every file either opens -- then every
tensor it lists reads back to host with the byte count its header gives --
or is rejected with SLTX_ERR_INVALID; hand-made cases must give their
expected outcome.  tests/test_sanitized.py reruns this file against the
AddressSanitizer / UndefinedBehaviorSanitizer build of the library.
"""
import json
import os

import pytest

CORPUS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "st_corpus")
EXPECT = json.load(open(os.path.join(CORPUS, "expect.json")))


@pytest.mark.parametrize("name", sorted(EXPECT))
def test_corpus_file(pkg, name):
    path = os.path.join(CORPUS, name + ".safetensors")
    want = EXPECT[name]
    try:
        f = pkg.SafeTensorsFile(path)
    except pkg.SltxError as e:
        assert e.code == pkg.SLTX_ERR_INVALID, (name, str(e))
        assert want != "ok", (name, str(e))
        if want is not None:
            assert want in str(e), (name, str(e))
        return
    assert want is None or want == "ok", (name, "opened, expected an error with", want)
    raw = open(path, "rb").read()
    for tname, info in f.tensors.items():
        a = f.read_host(tname)
        assert a.nbytes == info.byte_count
        hlen = int.from_bytes(raw[:8], "little")
        start = 8 + hlen + info.offset
        assert a.tobytes() == raw[start:start + info.byte_count], (name, tname)
    f.close()


def test_corpus_is_complete():
    files = {f[:-len(".safetensors")] for f in os.listdir(CORPUS) if f.endswith(".safetensors")}
    assert files == set(EXPECT)
    assert sum(v == "ok" for v in EXPECT.values()) >= 5
    assert sum(v is None for v in EXPECT.values()) >= 40
