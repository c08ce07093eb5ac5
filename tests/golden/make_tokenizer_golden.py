"""Golden token ids for the C++ tokenizer (ai_amd/host/tokenizer.cpp).

Builds two tokenizer.json files in the Gemma layout (byte-fallback BPE,
space -> metaspace Replace normalizer, Split pre-tokenizer, raw added tokens,
[BOS] A [EOS] template) and encodes test strings with Hugging Face
`tokenizers` (an independent implementation of that file format):
  * "small": the in-memory tokenizer of the reference's own test
    (tokenizer/synthetic_test.go:13-60), same vocab, merges and template;
  * "learned": ~300 merges learned here from a synthetic corpus over ASCII,
    accented Latin, Greek, CJK and emoji, plus added tokens embedded in text.
Writes tests/golden/tokenizer_golden.json: the files' text and, per case,
the string, Encode ids (template) and EncodeRaw ids. Run in the build
container: python tests/golden/make_tokenizer_golden.py
"""
import collections
import json
import os
import random

from tokenizers import Tokenizer

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tokenizer_golden.json")
META = "▁"


def doc(vocab, merges, added):
    return {
        "version": "1.0",
        "added_tokens": [{"id": vocab[a], "content": a, "single_word": False, "lstrip": False, "rstrip": False,
                          "normalized": False, "special": True} for a in added],
        "normalizer": {"type": "Replace", "pattern": {"String": " "}, "content": META},
        "pre_tokenizer": {"type": "Split", "pattern": {"String": " "}, "behavior": "MergedWithPrevious",
                          "invert": False},
        "post_processor": {
            "type": "TemplateProcessing",
            "single": [{"SpecialToken": {"id": "<bos>", "type_id": 0}}, {"Sequence": {"id": "A", "type_id": 0}},
                       {"SpecialToken": {"id": "<eos>", "type_id": 0}}],
            "pair": [{"Sequence": {"id": "A", "type_id": 0}}, {"Sequence": {"id": "B", "type_id": 1}}],
            "special_tokens": {"<bos>": {"id": "<bos>", "ids": [vocab["<bos>"]], "tokens": ["<bos>"]},
                               "<eos>": {"id": "<eos>", "ids": [vocab["<eos>"]], "tokens": ["<eos>"]}},
        },
        "decoder": None,
        "model": {"type": "BPE", "dropout": None, "unk_token": "<unk>", "continuing_subword_prefix": None,
                  "end_of_word_suffix": None, "fuse_unk": False, "byte_fallback": True, "ignore_merges": False,
                  "vocab": vocab, "merges": merges},
    }


def small():
    vocab = {"<pad>": 0, "<eos>": 1, "<bos>": 2, "<unk>": 3, META: 4, "a": 5, "b": 6, "c": 7, "ab": 8, "abc": 9,
             META + "a": 10}
    for b in range(256):
        vocab["<0x%02X>" % b] = 11 + b
    return doc(vocab, [["a", "b"], ["ab", "c"], [META, "a"]], ["<bos>", "<eos>", "<pad>"])


def learned(rng):
    alphabet = (list("abcdefghijklmnopqrstuvwxyz") + list("ABCDEFG0123456789.,:;-/") + list("éèüöñçß") +
                list("αβγδεζ") + list("中文字节") + ["\U0001F600"])
    words = ["".join(rng.choice(alphabet[:26]) for _ in range(rng.randint(2, 7))) for _ in range(60)]
    corpus = []
    for _ in range(4000):
        w = rng.choice(words) if rng.random() < 0.8 else "".join(rng.choice(alphabet) for _ in range(rng.randint(1, 5)))
        corpus.append(META + w)
    # base symbols: the alphabet except a few left to byte fallback
    base = [c for c in alphabet if c not in ("\U0001F600", "ß", "字")] + [META]
    seqs = [list(w) for w in corpus]
    merges = []
    pieces = set(base)
    for _ in range(300):
        cnt = collections.Counter()
        for s in seqs:
            for x, y in zip(s, s[1:]):
                if x in pieces and y in pieces:
                    cnt[(x, y)] += 1
        if not cnt:
            break
        (x, y), _ = max(cnt.items(), key=lambda kv: (kv[1], kv[0]))
        merges.append([x, y])
        pieces.add(x + y)
        for s in seqs:
            i = 0
            while i < len(s) - 1:
                if s[i] == x and s[i + 1] == y:
                    s[i:i + 2] = [x + y]
                i += 1
    added = ["<pad>", "<eos>", "<bos>", "<unk>", "<start_of_turn>", "<end_of_turn>", "<mask>"]
    vocab = {}
    for a in added:
        vocab[a] = len(vocab)
    for b in range(256):
        vocab["<0x%02X>" % b] = len(vocab)
    for p in sorted(pieces, key=lambda p: (len(p), p)):
        if p not in vocab:
            vocab[p] = len(vocab)
    return doc(vocab, merges, added), words, alphabet


def cases_for(rng, words, alphabet, n):
    out = ["", " ", "  ", "a", "The quick brown fox", "  leading and trailing  ", "<bos>", "x<start_of_turn>y",
           "<start_of_turn>user\nhello<end_of_turn>", "<mask><mask>", "<bo", "é ß 字 \U0001F600", "\t\n\r",
           "ab" * 40]
    for _ in range(n):
        parts = []
        for _ in range(rng.randint(1, 12)):
            r = rng.random()
            if r < 0.6:
                parts.append(rng.choice(words))
            elif r < 0.8:
                parts.append("".join(rng.choice(alphabet) for _ in range(rng.randint(1, 4))))
            elif r < 0.9:
                parts.append(rng.choice(["<start_of_turn>", "<end_of_turn>", "<mask>", "<bos>", "<eos>"]))
            else:
                parts.append(rng.choice(["ó", "Ω", " ", "😀x", "—", "ÿ"]))
        sep = rng.choice([" ", "  ", "", " "])
        out.append(sep.join(parts))
    return out


def main():
    rng = random.Random(20261201)
    docs = {"small": small()}
    ld, words, alphabet = learned(rng)
    docs["learned"] = ld
    files, cases = {}, []
    for name, d in docs.items():
        text = json.dumps(d, ensure_ascii=False)
        files[name] = text
        tok = Tokenizer.from_str(text)
        strings = (["abc", "ab", "ba", "a", " a", "", "Z", "é", "a<bos>b", "abc é"] if name == "small"
                   else cases_for(rng, words, alphabet, 120))
        for s in strings:
            cases.append({"tok": name, "s": s, "ids": tok.encode(s, add_special_tokens=True).ids,
                          "raw": tok.encode(s, add_special_tokens=False).ids})
    with open(OUT, "w", encoding="utf-8") as f:
        json.dump({"generator": "tokenizers " + __import__("tokenizers").__version__, "files": files,
                   "cases": cases}, f, ensure_ascii=False)
    print(f"wrote {OUT}: {len(cases)} cases, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
