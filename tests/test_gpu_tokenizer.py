"""The tokenizer bridge on the GPU box, end to end as tokenizer_test.mojo runs
it: text -> BPETokenizer ids -> the model on the device -> ids -> text.

- "Hallo Mojo" with the reference's vocab.msvocab encodes to [259, 32, 262]
  and decodes back (tokenizer_test.mojo:75; the hand derivation is in
  tests/test_tokenizer.py).
- Those ids prefill a 2-layer E4B-shape model with a 512-id tied head; its
  greedy ids equal the oracle's, and the tokenizer turns them into the text the
  restatement (oracle/tokenizer_ref.py) gives for the same ids.
- Random texts over the vocabulary's alphabet encode and decode as the
  restatement does.
"""
import os
import random

import numpy as np
import pytest

from oracle import tokenizer_ref as ref
from oracle.binding import Oracle, synthetic_oracle_model

pytestmark = pytest.mark.gpu
SEED = 42
GOLDEN_VOCAB = os.path.join(os.path.dirname(__file__), "golden", "vocab.msvocab")


def say(msg):
    print(f"\n[case] {msg}", flush=True)


def test_text_through_model_and_back(gpu):
    ms = gpu
    from mojostream_amd.tokenizer import BPETokenizer
    say("tokenizer bridge: 'Hallo Mojo' -> ids -> 2-layer model (vocab 512) -> ids -> text")
    tok = BPETokenizer(GOLDEN_VOCAB)
    vocab, id_to_tok, merges = ref.load(GOLDEN_VOCAB)
    ids = tok.encode("Hallo Mojo")
    assert ids == [259, 32, 262] == ref.encode(b"Hallo Mojo", merges, vocab)
    assert tok.decode(ids) == "Hallo Mojo"
    arch = ms.arch_e4b(max_full_seq=64, n_layers=2, vocab=512)
    m = ms.Model(arch, max_seqs=1, max_rows=4, max_pos=64)
    m.fill_synthetic(SEED, balanced=True)
    m.set_sampling(0.0, 1.2, 0)          # greedy over the penalized logits
    steps = 8
    first = m.prefill(ids, 0)
    out = [first] + [int(v) for v in m.decode([first], [len(ids)], steps - 1)[:, 0]]
    m.close()
    o = Oracle()
    om = synthetic_oracle_model(o, arch, SEED, balanced=True)
    hist = list(ids)
    x = None
    for p, t in enumerate(ids):
        _, x = om.decode_token(t, p, hidden=True)
    want = []
    for k in range(steps):
        if k:
            _, x = om.decode_token(want[-1], len(ids) + k - 1, hidden=True)
        tid, _ = o.sample(om.logits_for(x[-1]), 0.0, hist, 1.2, 0)
        want.append(tid)
        hist.append(tid)
    text = tok.decode(out)
    print(f"  device ids {out} -> {text!r}\n  oracle ids {want}")
    assert out == want
    assert text == ref.decode(out, id_to_tok).decode("latin-1")
    assert [tok.token_str(i) for i in out] == [
        (id_to_tok[i] if 0 <= i < len(id_to_tok) else b"<unk>").decode("latin-1") for i in out]
    tok.close()


def test_random_texts_vs_restatement(gpu):
    from mojostream_amd.tokenizer import BPETokenizer
    say("tokenizer: 300 random texts over the reference vocabulary vs the restatement")
    tok = BPETokenizer(GOLDEN_VOCAB)
    vocab, id_to_tok, merges = ref.load(GOLDEN_VOCAB)
    rng = random.Random(11)
    alpha = b"HaloMj lo"
    for _ in range(300):
        text = bytes(rng.choice(alpha) for _ in range(rng.randint(0, 40)))
        got = tok.encode(text.decode())
        assert got == ref.encode(text, merges, vocab)
        assert tok.decode(got) == ref.decode(got, id_to_tok).decode("latin-1")
    tok.close()
