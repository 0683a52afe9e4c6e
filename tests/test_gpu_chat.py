"""The chat driver (main.rs:28-158) on the GPU with a word-level tokenizer over a tiny hybrid
model: the first reply is the oracle's greedy continuation of the ChatML turn up to the stop id,
<|im_end|> is forwarded, and the second reply is the oracle's continuation of the whole
conversation as the reference's cache holds it (turn 1, reply 1, <|im_end|>, turn 2)."""
import numpy as np
import pytest

import oracle as O
import q35
from q35.chat import ChatSession, chatml_turn
from test_chat import word_tokenizer

pytestmark = pytest.mark.gpu


def hybrid_dims():
    return q35.make_dims(hidden=512, ffn=1536, vocab=8192, n_layers=4, lin_heads=4, attn_heads=4, kv_heads=2)


def oracle(d, seed, tmax):
    return O.Model(O.cfg_from_dims(d), lambda name, n: q35.synth_model_tensor(d, seed, name, n), tmax)


@pytest.mark.parametrize("chunk,stream", [(4, False), (32, False), (32, True)])
def test_chat_session_matches_oracle_conversation(chunk, stream):
    """Two turns against the oracle, the reply in launches of `chunk` steps or streamed."""
    print(f"[chat] chunk={chunk} stream={stream}", flush=True)
    d, seed, tmax = hybrid_dims(), 3, 256
    im_end = 7
    tok = word_tokenizer(d.vocab, im_end=im_end, im_start=9)
    turn1 = tok.encode(chatml_turn("hello world", True), add_special_tokens=False).ids
    rt, _ = oracle(d, seed, tmax).generate(np.array(turn1, np.int32), 40)
    k = next(j for j in range(3, 40) if rt[j] not in set(rt[:j].tolist()) and rt[j] != im_end)
    eos = int(rt[k])
    m = q35.TextForCausalLM(d, seed=seed, tmax=tmax)
    chat = ChatSession(m, tok, max_output_tokens=30, eos_id=eos, chunk=chunk, stream=stream)
    r1 = chat.send("hello world")
    assert r1.stopped and r1.ids == [int(t) for t in rt[:k]]
    assert r1.text == tok.decode(r1.ids, skip_special_tokens=True)
    assert m.position() == len(turn1) + k + 1
    turn2 = tok.encode(chatml_turn("again", False), add_special_tokens=False).ids
    conv = np.array(turn1 + r1.ids + [im_end] + turn2, np.int32)
    rt2, _ = oracle(d, seed, tmax).generate(conv, 10)
    want = []
    for t in rt2[:10]:
        if t in (im_end, eos):
            break
        want.append(int(t))
    r2 = chat.send("again")
    r2_ids = r2.ids[:10]
    assert r2_ids[:len(want)] == want
    assert r2.ctx_tokens == len(conv) + len(r2.ids) + 1
    m.close()
