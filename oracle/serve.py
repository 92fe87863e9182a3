"""The reference's --serve loop restated (src/qwythos.cpp: protocol qw:2139-2148, serve_loop qw:2593-2813, topk_out
qw:2513-2531), over an abstract engine, to check the engine's rmi_serve_fd / rmi_serve_engine line by line.

TEST INFRASTRUCTURE ONLY (the checker of the serving protocol).

The engine object provides:
    max_ctx                     context length
    reset()                     empty context, position 0
    position() -> int           tokens in the context
    ingest(tokens) -> int       feed tokens at the current position; the greedy token after them
    top(k) -> [(id, logit)]     the k largest logits that chose the current token (k > 0)
    greedy_step() -> int        feed the current token; the greedy token after it
    mtp_begin()                 the first draft candidate of the current token
    mtp_round() -> (c0, c1, accepted)   one verify round (feeds 2 tokens on accept, 1 on reject)

Requests are read as the reference reads them (substring matches on the compact JSON the server sends:
qw:2622-2660); "topk":K is this engine's addition (the reference always lists 40).
"""
from __future__ import annotations

EOS = 248046   # serve_loop's end-of-turn id (qw:2752, 2765, 2807)


def _num_in(line: str, key: str) -> int:
    """num_in (qw:2625-2630): atoll of what follows "key":, -1 when absent"""
    pat = '"' + key + '":'
    at = line.find(pat)
    if at < 0:
        return -1
    s = line[at + len(pat):].lstrip(" \t\n\r\f\v")
    j = 0
    if j < len(s) and s[j] in "+-":
        j += 1
    while j < len(s) and s[j].isdigit():
        j += 1
    try:
        return int(s[:j])
    except ValueError:
        return 0


def _tokens(line: str) -> list:
    """the digit scan of qw:2644-2656"""
    toks = []
    at = line.find('"tokens":[')
    if at < 0:
        return toks
    v, inn, neg = 0, False, False
    for ch in line[at + 10:]:
        if ch == "]":
            break
        if ch == "-":
            neg = True
            continue
        if ch.isdigit():
            v = v * 10 + int(ch)
            inn = True
            continue
        if inn:
            toks.append(-v if neg else v)
            v, inn, neg = 0, False, False
    if inn:
        toks.append(-v if neg else v)
    return toks


def token_line(tid: int, top) -> str:
    """topk_out's line (qw:2505-2531): {"id":I,"top":[[id,%.5f],..]}"""
    return '{"id":%d,"top":[%s]}' % (tid, ",".join("[%d,%.5f]" % (i, v) for i, v in top))


def serve(engine, lines, eos: int = EOS, topk: int = 40):
    """the response lines for the request lines"""
    out = []
    for line in lines:
        if line == "":
            continue
        if '"op":"reset"' in line:                                   # qw:2632-2641
            engine.reset()
            out.append('{"ok":true,"op":"reset"}')
            continue
        gen = _num_in(line, "gen")
        mtp = '"mtp":true' in line
        toks = _tokens(line)
        k = _num_in(line, "topk") if '"topk":' in line else topk
        if not toks or gen <= 0:                                     # qw:2657-2661
            out.append('{"error":"need tokens and gen"}')
            continue
        pos = engine.position()
        if pos + len(toks) + gen + 8 >= engine.max_ctx:               # qw:2662-2666
            out.append('{"error":"context full; send op reset"}')
            continue
        cur = engine.ingest(toks)                                    # qw:2670-2738

        def emit_top(tid):
            out.append(token_line(tid, engine.top(k) if k > 0 else []))

        if not mtp:                                                  # qw:2748-2759
            emitted = 0
            while emitted < gen:
                emit_top(cur)
                emitted += 1
                if cur == eos:
                    break
                cur = engine.greedy_step()
            out.append('{"done":true,"pos":%d}' % engine.position())
            continue
        emit_top(cur)                                                # qw:2761-2809
        emitted = 1
        if cur != eos and emitted < gen:
            engine.mtp_begin()
            while emitted < gen:
                c0, c1, accepted = engine.mtp_round()
                out.append(token_line(c0, []))
                emitted += 1
                if accepted:
                    if emitted < gen:
                        out.append(token_line(c1, []))
                        emitted += 1
                        cur = c1
                    else:
                        cur = c0
                else:
                    cur = c0
                if cur == eos:
                    break
        out.append('{"done":true,"pos":%d}' % engine.position())
    return out
