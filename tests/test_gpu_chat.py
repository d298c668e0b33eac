"""The chat turn logic (cuqwen_amd.ChatSession, the reference's chat loop
src/main.cu:40-126) on the device against the host oracle: templated and
tokenized turns, prefill, greedy decode with the turn's generated ids as the
penalty history, stop ids, and the second turn continuing at the next
position with only the new turn templated."""
import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.conftest import tiny_config
from tests.test_tokenizer import train_hf_tokenizer, write_ranks

pytestmark = pytest.mark.gpu


def _oracle_turn(om, prompt, pos, stop, max_new):
    nxt = None
    for i, t in enumerate(prompt):
        nxt = om.forward(t, pos + i, [])
    pos += len(prompt)
    gen, near_tie = [], False
    while nxt not in stop and len(gen) < max_new:
        gen.append(nxt)
        l = np.sort(om.logits().astype(np.float64))
        near_tie |= l[-1] - l[-2] <= 1e-2
        nxt = om.forward(nxt, pos, gen)
        pos += 1
    return gen, pos, near_tie


def test_chat_session_two_turns_match_oracle(tmp_path):
    hf = train_hf_tokenizer()
    path = tmp_path / "ranks.json"
    write_ranks(hf, path)
    tok = cq.Tokenizer(str(path))
    cfg = tiny_config(2)
    w = cq.synth_weights(cfg, 11)
    st = cq.State(cfg, w)
    eos, im_end = tok.token_id("<|endoftext|>"), tok.token_id("<|im_end|>")
    chat = cq.ChatSession(st, tok, eos_id=eos, im_end_id=im_end)
    om = orc.Model.synth(cfg, 11, cfg.max_seq_len)
    pos, compared = 0, 0
    turns = ["Hello there! How's it going?", "Tell me about 日本語 and numbers 42."]
    for k, user in enumerate(turns):
        msgs = [("user", user)]
        prompt = tok.encode(cq.Tokenizer.apply_chat_template(msgs, True))
        assert prompt[0] == tok.token_id("<|im_start|>")
        text, gen = chat.reply(user, max_new_tokens=12)
        want, pos, near_tie = _oracle_turn(om, prompt, pos, (eos, im_end), 12)
        if not near_tie:
            assert gen == want, k
            compared += 1
        assert text == tok.decode(gen)
        assert chat.pos == pos
    assert compared >= 1
    assert [r for r, _ in chat.history] == ["user", "assistant", "user", "assistant"]
    st.free()
    w.free()
    tok.free()


def test_chat_cli_matches_chat_session(tmp_path):
    """python -m cuqwen_amd.chat (the reference's REPL, src/main.cu:14-140):
    two user turns on stdin, then "exit"; the streamed replies equal
    ChatSession's on the same weights, and each turn ends with the
    reference's stats line."""
    import subprocess
    import sys
    hf = train_hf_tokenizer()
    ranks = tmp_path / "ranks.json"
    write_ranks(hf, ranks)
    cfg = tiny_config(2)
    wpath = str(tmp_path / "tiny.bin")
    cq.write_synthetic_file(wpath, cfg, 11)
    turns = ["Hello there! How's it going?", "", "Tell me about 日本語 and numbers 42."]
    r = subprocess.run([sys.executable, "-m", "cuqwen_amd.chat", "--weights", wpath, "--tokenizer", str(ranks),
                        "--max-new-tokens", "10"], input=("\n".join(turns + ["exit"]) + "\n").encode(),
                       capture_output=True, timeout=300,
                       cwd=str(tmp_path), env=dict(__import__("os").environ, PYTHONPATH=cq._HERE + "/.."))
    assert r.returncode == 0, r.stderr.decode(errors="replace")
    tok = cq.Tokenizer(str(ranks))
    cfg2, w = cq.load_weights(wpath)
    st = cq.State(cfg2, w)
    chat = cq.ChatSession(st, tok, eos_id=tok.token_id("<|endoftext|>"), im_end_id=tok.token_id("<|im_end|>"))
    gens = [chat.reply(t, max_new_tokens=10)[1] for t in turns if t]
    out = r.stdout   # bytes: a random-weight reply need not be valid UTF-8
    for gen in gens:
        assert b"Qwen > " + tok.decode_bytes(gen) + b"\n\n[" in out
    assert out.count(b"tokens generated |") == 2
    assert f"Context: {chat.pos}/{cfg.max_seq_len}]".encode() in out
    st.free()
    w.free()
    tok.free()
