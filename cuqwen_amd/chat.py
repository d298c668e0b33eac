"""Interactive chat on the engine: the reference's chat REPL (src/main.cu:14-140)
as a command-line program over cuqwen_amd.ChatSession.

    python -m cuqwen_amd.chat --weights weights/model_int4_7b.bin \\
        --tokenizer weights/qwen25_bpe_ranks.json

Reads user turns from stdin ("exit" or "quit" or end of input stops), streams
the reply token by token to stdout, and prints the reference's per-turn line
"[N tokens generated | X tok/s | Context: pos/max]".  The first turn sends the
whole templated conversation, later turns only the new user turn; decode is
greedy with the turn's generated ids as the repetition-penalty history and
stops at <|endoftext|> / <|im_end|> or at max_seq_len - 2, as in the
reference.  The prompt goes through the batched prefill (the reference runs
one decode step per prompt token; the greedy result is the same).
"""
import argparse
import os
import sys
import time

EOS_ID, IM_END_ID = 151643, 151645   # src/main.cu:24-25


def main(argv=None, stdin=None, stdout=None):
    ap = argparse.ArgumentParser(prog="python -m cuqwen_amd.chat", description=__doc__.split("\n\n")[0])
    ap.add_argument("--weights", required=True, help="weight file in the exporter's layout (export_weights.py)")
    ap.add_argument("--tokenizer", default=os.path.join("weights", "qwen25_bpe_ranks.json"),
                    help="tokenizer ranks file (export_weights.py export_tokenizer)")
    ap.add_argument("--kv-cache", choices=["fp16", "int8", "fp8"], default="fp16")
    ap.add_argument("--max-new-tokens", type=int, default=None, help="cap per reply (default: up to the stop ids)")
    args = ap.parse_args(argv)
    stdin = stdin or sys.stdin
    out = stdout or sys.stdout
    bout = getattr(out, "buffer", None)

    def say(text, end="\n"):
        out.write(text + end)
        out.flush()

    for path, what in ((args.weights, "weight file"), (args.tokenizer, "tokenizer file")):
        if not os.path.exists(path):
            print(f"chat: {what} {path} not found", file=sys.stderr)
            return 1
    import cuqwen_amd as cq

    say("=" * 72)
    say("         cuqwen_amd chat (MI355X batch-1 Qwen2.5 decode engine)")
    say("=" * 72)
    say(f"[*] Loading tokenizer from: {args.tokenizer}...", end="")
    tok = cq.Tokenizer(args.tokenizer)
    say(" Done.")
    say(f"[*] Loading weights from: {args.weights}...", end="")
    cfg, w = cq.load_weights(args.weights)
    kv = {"fp16": cq.KV_FP16, "int8": cq.KV_INT8, "fp8": cq.KV_FP8}[args.kv_cache]
    st = cq.State(cfg, w, kv)
    say(" Done.")
    eos = tok.token_id("<|endoftext|>")
    im_end = tok.token_id("<|im_end|>")
    chat = cq.ChatSession(st, tok, eos_id=eos if eos >= 0 else EOS_ID, im_end_id=im_end if im_end >= 0 else IM_END_ID)
    limit = cfg.max_seq_len - 2
    say("[+] Engine initialized. Type 'exit' or 'quit' to end the session.")
    say("=" * 72)

    def emit(token_id):
        piece = tok.decode_bytes([token_id])
        if bout is not None:
            out.flush()
            bout.write(piece)
            bout.flush()
        else:
            out.write(piece.decode("utf-8", errors="replace"))
            out.flush()

    try:
        while True:
            if chat.pos >= limit:
                say(f"\n[!] Context window fully used ({chat.pos}/{cfg.max_seq_len}). Ending the session.")
                break
            say("\nUser > ", end="")
            line = stdin.readline()
            if not line:
                break
            user = line.rstrip("\r\n")
            if user in ("exit", "quit"):
                break
            if not user:
                continue
            say("Qwen > ", end="")
            t0 = time.perf_counter()
            try:
                _, gen = chat.reply(user, max_new_tokens=args.max_new_tokens, on_token=emit)
            except cq.CuQwenError as e:
                if e.code == 6:   # CQ_ERANGE: the prompt does not fit the remaining context
                    say(f"\n[!] Prompt too long for the remaining context ({chat.pos}/{cfg.max_seq_len}). "
                        "Ending the session.")
                    break
                raise
            dt = time.perf_counter() - t0
            rate = len(gen) / dt if gen and dt > 0 else 0.0
            say(f"\n\n[{len(gen)} tokens generated | {rate:.2f} tok/s | Context: {chat.pos}/{cfg.max_seq_len}]")
    finally:
        st.free()
        w.free()
        tok.free()
    return 0


if __name__ == "__main__":
    sys.exit(main())
