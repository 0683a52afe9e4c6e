"""CPU tests of the chat driver (main.rs:28-158) with a scripted stand-in for the model: the
ChatML turn texts, the stop on <|im_end|> / eos (also when it falls on a chunk boundary), the
max_output_tokens limit, <|im_end|> forwarded after each reply, the context count, /reset, and
the incremental detokenisation that holds back an incomplete UTF-8 tail."""
import pytest
from tokenizers import AddedToken, Tokenizer, models, pre_tokenizers

from q35.chat import EOS_ID, ChatSession, StreamDecoder, chatml_turn


def test_chatml_turn_texts():
    assert chatml_turn("hi", True) == ("<|im_start|>system\nYou are a helpful assistant.<|im_end|>\n"
                                       "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n")
    assert chatml_turn("again", False) == "\n<|im_start|>user\nagain<|im_end|>\n<|im_start|>assistant\n"
    assert chatml_turn("x", True, system="S").startswith("<|im_start|>system\nS<|im_end|>")


class ByteTok:
    """Ids are byte values; decode is UTF-8 with U+FFFD for an incomplete sequence."""

    def decode(self, ids, skip_special_tokens=True):
        return bytes(ids).decode("utf-8", errors="replace")


def test_stream_decoder_holds_back_incomplete_utf8():
    text = "añ€𝄞b"
    ids = list(text.encode("utf-8"))
    sd = StreamDecoder(ByteTok())
    pieces = [sd.push([i]) for i in ids]
    assert "".join(pieces) + sd.tail() == text
    assert all("�" not in p for p in pieces)
    # the 4-byte clef only appears once its last byte arrived
    start = len("añ€".encode())
    assert pieces[start:start + 3] == ["", "", ""] and pieces[start + 3] == "𝄞"


def word_tokenizer(vocab_size, im_end, im_start):
    words = ["system", "user", "assistant", "You", "are", "a", "helpful", ".", "hello", "world", "again"]
    vocab = {f"w{i}": i for i in range(vocab_size)}
    for i, w in enumerate(words):
        del vocab[f"w{100 + i}"]
        vocab[w] = 100 + i
    for tok, i in (("<|im_end|>", im_end), ("<|im_start|>", im_start)):
        del vocab[f"w{i}"]
        vocab[tok] = i
    t = Tokenizer(models.WordLevel(vocab, unk_token="w0"))
    t.pre_tokenizer = pre_tokenizers.Whitespace()
    t.add_special_tokens([AddedToken("<|im_end|>", special=True), AddedToken("<|im_start|>", special=True)])
    return t


class ScriptModel:
    """decode_until replays a scripted greedy sequence; records what the session fed."""

    def __init__(self, script, tmax=1 << 20):
        self.script, self.i = list(script), 0
        self.prefills, self.forwarded, self.resets = [], [], 0
        self.tmax, self.pos, self.max_asked = tmax, 0, 0

    def position(self):
        return self.pos

    def prefill(self, ids):
        assert self.pos + len(ids) <= self.tmax, "prefill past tmax"
        self.prefills.append(list(ids))
        self.pos += len(ids)

    def decode_until(self, n, stop_ids=(), mode=None):
        # as q35_model_decode_until: refused unless position + n fits the cache
        assert self.pos + n <= self.tmax, "decode_until past tmax"
        self.max_asked = max(self.max_asked, n)
        out = []
        while len(out) < n:
            t = self.script[self.i]
            if t in stop_ids:
                self.pos += len(out)
                return out, t, 0.0
            out.append(t)
            self.i += 1
        self.pos += len(out)
        return out, self.script[self.i], 0.0

    def set_token(self, t):
        self.forwarded.append(t)

    def step(self, mode=None):
        assert self.pos < self.tmax, "step past tmax"
        self.pos += 1
        self.i += 1 if self.forwarded and self.script[self.i] == self.forwarded[-1] else 0

    def reset(self):
        self.resets += 1
        self.pos = 0


class StreamScriptModel(ScriptModel):
    """The same script through current_token / decode_stream (the streamed reply path)."""

    def current_token(self):
        return self.script[self.i]

    def decode_stream(self, n, stop_ids=()):
        # as q35_model_decode_stream: refused unless position + n fits the cache; the launch
        # ends before a step whose input token is a stop id; each step yields its argmax
        assert self.pos + n <= self.tmax, "decode_stream past tmax"
        self.max_asked = max(self.max_asked, n)
        for _ in range(n):
            if self.script[self.i] in stop_ids:
                return
            self.i += 1
            self.pos += 1
            yield self.script[self.i]


FAKES = {"chunked": ScriptModel, "streamed": StreamScriptModel}


@pytest.mark.parametrize("fake", ["chunked", "streamed"])
@pytest.mark.parametrize("chunk", [1, 3, 4, 32])
def test_session_stops_and_forwards_im_end(chunk, fake):
    tok = word_tokenizer(1024, im_end=7, im_start=9)
    reply1 = [500, 501, 502, 503]  # 4 ids, then <|im_end|> (a chunk boundary when chunk is 4)
    m = FAKES[fake](reply1 + [7] + [600, 601, EOS_ID])
    s = ChatSession(m, tok, chunk=chunk)
    r = s.send("hello world")
    assert r.ids == reply1 and r.stopped
    assert m.prefills[0] == tok.encode(chatml_turn("hello world", True), add_special_tokens=False).ids
    assert m.forwarded == [7]
    assert r.ctx_tokens == len(m.prefills[0]) + len(reply1) + 1
    r2 = s.send("again")
    assert m.prefills[1] == tok.encode(chatml_turn("again", False), add_special_tokens=False).ids
    assert r2.ids == [600, 601] and r2.stopped  # eos ends it too
    assert m.forwarded == [7, 7]
    assert r2.ctx_tokens == r.ctx_tokens + len(m.prefills[1]) + 2 + 1
    s.reset()
    assert m.resets == 1 and s.turns == 0 and s.total_tokens == 0
    m.i = 0
    s.send("hello")
    assert m.prefills[2][:3] == m.prefills[0][:3]  # the system prompt again


@pytest.mark.parametrize("fake", ["chunked", "streamed"])
def test_session_max_output_tokens(fake):
    tok = word_tokenizer(1024, im_end=7, im_start=9)
    m = FAKES[fake](list(range(200, 260)) + [7])
    s = ChatSession(m, tok, max_output_tokens=10, chunk=4)
    r = s.send("hello")
    assert r.ids == list(range(200, 210)) and not r.stopped
    assert m.forwarded == [7]


@pytest.mark.parametrize("fake", ["chunked", "streamed"])
def test_session_stays_inside_the_cache(fake):
    """Near tmax the reply is cut so that the <|im_end|> forward still has a row (no call asks
    for more rows than are left), and a turn that does not fit is reported as a full context
    without touching the model; /reset makes room again."""
    tok = word_tokenizer(1024, im_end=7, im_start=9)
    turn_len = len(tok.encode(chatml_turn("hello world", True), add_special_tokens=False).ids)
    tmax = turn_len + 10
    m = FAKES[fake](list(range(200, 260)) + [7], tmax=tmax)
    s = ChatSession(m, tok, chunk=4)
    r = s.send("hello world")
    assert r.context_full and not r.stopped
    assert r.ids == list(range(200, 209))  # 10 free rows: 9 reply ids, 1 row for <|im_end|>
    assert m.forwarded == [7] and m.position() == tmax
    r2 = s.send("again")
    assert r2.context_full and r2.ids == [] and len(m.prefills) == 1
    s.reset()
    m.i = 0
    r3 = s.send("hello world")
    assert r3.ids == list(range(200, 209)) and len(m.prefills) == 2
