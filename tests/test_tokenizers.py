"""The library's tokenizers (tsn_clip_tokenizer_*, tsn_t5_tokenizer_*: ClipTokenizer and
T5Tokenizer, src/tokenizers.cpp) against the oracle's restatement (oracle/pyoracle.py), with
vocabularies written into tokenizer GGUFs as array metadata the way the reference reads them
(clip.vocab / clip.merges / clip.bos_id / clip.eos_id, t5.pieces / t5.scores / t5.*_id) — CPU only.

Texts cover upper case, tabs and newlines, repeated and trailing spaces, UTF-8 multi-byte
characters, characters outside the vocabulary, and texts longer than the context (truncation
with eos last) and shorter (eos or pad padding).
"""
import numpy as np
import pytest

from conftest import rng
from gguf_writer import KV_ARRAY, KV_F32, KV_STRING, KV_U32, F32, write


def _train_bpe(words, n_merges, bsym):
    """a small BPE merge list from word frequencies (the test's own vocabulary)"""
    corpus = [[bsym[b] for b in w.encode()] for w in words]
    for w in corpus:
        w[-1] += "</w>"
    merges = []
    for _ in range(n_merges):
        counts = {}
        for w in corpus:
            for a, b in zip(w, w[1:]):
                counts[(a, b)] = counts.get((a, b), 0) + 1
        if not counts:
            break
        (a, b), _ = max(counts.items(), key=lambda kv: (kv[1], kv[0]))
        merges.append(a + " " + b)
        for w in corpus:
            i = 0
            while i + 1 < len(w):
                if w[i] == a and w[i + 1] == b:
                    w[i:i + 2] = [a + b]
                i += 1
    return merges


@pytest.fixture(scope="module")
def clip_tok(tsn, orc, tmp_path_factory):
    bsym = orc._byte_symbols()
    r = rng(1)
    words = ["".join(r.choice(list("abcdeghlnorst"), size=r.integers(1, 8))) for _ in range(300)]
    merges = _train_bpe(words, 120, bsym)
    vocab = list(bsym.values()) + [v + "</w>" for v in bsym.values()] + [m.replace(" ", "") for m in merges]
    path = str(tmp_path_factory.mktemp("tok") / "clip-tokenizer.gguf")
    write(path, [("x", (4,), F32, np.zeros(4, np.float32))],
          [("clip.vocab", KV_ARRAY, (KV_STRING, vocab)), ("clip.merges", KV_ARRAY, (KV_STRING, merges)),
           ("clip.bos_id", KV_U32, 49406), ("clip.eos_id", KV_U32, 49407)])
    t = tsn.ClipTokenizer(path)
    yield t, vocab, merges
    t.close()


@pytest.fixture(scope="module")
def t5_tok(tsn, tmp_path_factory):
    r = rng(2)
    alphabet = list("▁abcdelnorst") + ["é", "ü"]
    pieces = ["<pad>", "</s>", "<unk>"] + sorted({"".join(r.choice(alphabet, size=k)) for k in (1, 1, 2, 3, 4)
                                                  for _ in range(60)})
    scores = [0.0, 0.0, 0.0] + [float(x) for x in -r.uniform(2, 12, size=len(pieces) - 3)]
    path = str(tmp_path_factory.mktemp("tok") / "t5-tokenizer.gguf")
    write(path, [("x", (4,), F32, np.zeros(4, np.float32))],
          [("t5.pieces", KV_ARRAY, (KV_STRING, pieces)), ("t5.scores", KV_ARRAY, (KV_F32, scores)),
           ("t5.unk_id", KV_U32, 2), ("t5.eos_id", KV_U32, 1), ("t5.pad_id", KV_U32, 0)])
    t = tsn.T5Tokenizer(path)
    yield t, pieces, scores
    t.close()


def _texts(seed, alphabet):
    r = rng(seed)
    out = ["", " ", "  lead and trail  ", "UPPER lower\tTab\nNewline", "a" * 200]
    for _ in range(60):
        out.append("".join(r.choice(alphabet, size=r.integers(1, 40))))
    return out


def test_clip_tokenizer_matches_oracle(orc, clip_tok):
    t, vocab, merges = clip_tok
    for text in _texts(3, list("abcdeghlnorstABCX  \t\n!é")):
        for ctx in (77, 8):
            want = orc.clip_bpe_encode(vocab, merges, text, ctx)
            assert t.encode(text, ctx) == want, (text, ctx)
    ids = t.encode("Hello there", 77)
    assert ids[0] == 49406 and len(ids) == 77 and ids[-1] == 49407


def test_t5_tokenizer_matches_oracle(orc, t5_tok):
    t, pieces, scores = t5_tok
    for text in _texts(4, list("abcdelnorstxyz  é\tü")):
        for ctx, pad in ((77, True), (77, False), (6, True)):
            want = orc.t5_unigram_encode(pieces, scores, text, ctx, pad)
            assert t.encode(text, ctx, pad) == want, (text, ctx, pad)
    ids = t.encode("a b", 77, True)
    assert len(ids) == 77 and ids[-1] == 0 and 1 in ids


def test_tokenizer_load_errors(tsn, tmp_path):
    path = str(tmp_path / "empty.gguf")
    write(path, [("x", (4,), F32, np.zeros(4, np.float32))])
    with pytest.raises(RuntimeError):
        tsn.ClipTokenizer(path)
    with pytest.raises(RuntimeError):
        tsn.T5Tokenizer(path)
