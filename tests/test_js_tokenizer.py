"""The JS host's tokenizer (tabinfer_amd/host/tokenizer.js; models/qwen3.js:3227-3320) against
Hugging Face `tokenizers` (an independent implementation of the same byte-level BPE) on a
tokenizer.json built here with Qwen's pre-tokenizer: a Split on Qwen's regex, then the
ByteLevel byte map, BPE merges trained on this repository's text plus mixed-script lines,
and the ChatML special tokens.

Pinned: the ids of fixed and seeded random strings (contractions in either case, digit
runs, whitespace and newline runs, CJK, emoji, accents, code), decode round trips and the
streamed pieces (a character whose bytes span two tokens comes out once, whole), the
ChatML prompt against the library encoding the same prompt with its special tokens, the
stop ids, both merge spellings ("a b" and ["a", "b"]), and the built-in Qwen pattern when a
file carries no Split pre-tokenizer.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import Regex, Tokenizer, decoders, models, pre_tokenizers, trainers  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SPEC = os.path.join(HERE, "js", "tok_spec.js")
QWEN = r"""(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+"""
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]

pytestmark = pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")

FIXED = ["Hello world", "I'LL don't we've THEY'RE it's O'Neil", "12345 + 67.89 = 1e-3", "  leading\n\n\ttabs   and  spaces  \n",
         "你好，世界！ こんにちは 🙂🚀", "naïve café — «quotes» ½ ∑", "def f(x):\n    return x**2  # comment\n", "", " ", "\n",
         "a\r\nb", "!!!???...", "x y z", "Ωμέγα Ελληνικά", "emoji 👩‍💻 zwj", "tab\tend\t", "'s's'S", "1234567890"]


def random_texts(n, seed):
    rng = np.random.default_rng(seed)
    pool = list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789    \n\t'.,;:!?-_()[]{}\"/\\") + \
        list("éüßñçøåœ你好世界日本語한국어🙂🚀½∑Ωμ") + ["'s", "'T", "'re", "'VE", "'ll", "'d", "\r\n", "  ", "\n\n"]
    return ["".join(rng.choice(pool, size=int(rng.integers(0, 40)))) for _ in range(n)]


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([pre_tokenizers.Split(Regex(QWEN), behavior="isolated", invert=False),
                                                 pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    corpus = [open(os.path.join(ROOT, f), encoding="utf-8").read() for f in ("DESIGN.md", "INTEGRATION.md")]
    corpus += ["Bonjour, ça va? Ich heiße Jürgen. 你好，世界！ こんにちは 🙂🚀 — naïve café 한국어 Ωμέγα"] * 64
    tr = trainers.BpeTrainer(vocab_size=3000, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                             special_tokens=SPECIALS, show_progress=False)
    tok.train_from_iterator(corpus, tr)
    d = tmp_path_factory.mktemp("tok")
    tok.save(str(d / "tokenizer.json"))
    return tok, d


def run_js(tokdir, texts, chats=()):
    spec = os.path.join(tokdir, "spec.json")
    with open(spec, "w") as f:
        json.dump({"tokenizer": str(tokdir), "texts": texts, "chats": list(chats)}, f)
    r = subprocess.run(["node", SPEC, spec], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


def test_ids_match_the_library(built):
    tok, d = built
    texts = FIXED + random_texts(300, 7)
    out = run_js(d, texts)
    for t, ids in zip(texts, out["ids"]):
        assert ids == tok.encode(t).ids, repr(t)
    assert out["dec"] == texts                       # byte-level BPE is lossless
    # streamed: the pieces join to the text, and no piece holds half a character
    for t, parts in zip(texts, out["stream"]):
        assert "".join(parts) == t
        assert all("\ufffd" not in p for p in parts) or "\ufffd" in t
    # (an empty piece before the end: a token that ended inside a character)
    assert any(p == "" for parts in out["stream"] for p in parts[:-1]), "no character spans two tokens here"


def test_chatml_prompt_and_stop_ids(built):
    tok, d = built
    chats = [[{"role": "system", "content": "You are helpful."}, {"role": "user", "content": "Hi there!"}],
             [{"role": "user", "content": "多行\n文本 and 'quotes'"}, {"role": "assistant", "content": "ok"},
              {"role": "user", "content": ""}]]
    out = run_js(d, [], chats)
    for msgs, got, got_ng in zip(chats, out["chat"], out["chatNoGen"]):
        body = "".join("<|im_start|>%s\n%s<|im_end|>\n" % (m["role"], m["content"]) for m in msgs)
        assert got_ng == tok.encode(body).ids
        assert got == tok.encode(body + "<|im_start|>assistant\n").ids
    assert out["stop"] == sorted([tok.token_to_id("<|im_end|>"), tok.token_to_id("<|endoftext|>")])


def test_merge_spellings_and_default_pattern(built, tmp_path):
    tok, d = built
    j = json.load(open(os.path.join(d, "tokenizer.json"), encoding="utf-8"))
    texts = FIXED + random_texts(60, 11)
    want = [tok.encode(t).ids for t in texts]
    # merges written as "a b" strings instead of pairs (or the reverse)
    m = j["model"]["merges"]
    j["model"]["merges"] = [" ".join(x) for x in m] if isinstance(m[0], list) else [x.split(" ", 1) for x in m]
    (tmp_path / "a").mkdir()
    json.dump(j, open(tmp_path / "a" / "tokenizer.json", "w", encoding="utf-8"))
    assert run_js(tmp_path / "a", texts)["ids"] == want
    # no Split in the file: the built-in Qwen pattern is the same one
    j["pre_tokenizer"] = {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False}
    (tmp_path / "b").mkdir()
    json.dump(j, open(tmp_path / "b" / "tokenizer.json", "w", encoding="utf-8"))
    assert run_js(tmp_path / "b", texts)["ids"] == want
