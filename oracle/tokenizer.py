"""CPU oracle for the GPT-2 text tokenizer -- TEST INFRASTRUCTURE ONLY.

A plain-Python restatement of the reference's tokenizer (tokenizer.c), used
by tests/ as the reference for the library's g2_tok_* entry points; nothing in
the product path imports it.  Each function cites the lines it follows.

Pinned by (tests/test_tokenizer.py): golden vectors written by the
reference's own tokenizer.c built from its sources (oracle/Makefile, target
`ref`; tests/golden/make_tokenizer_fixture.py), the same comparison live
against that build when it is present, the byte alphabet and the merge
procedure against HF transformers' GPT2Tokenizer on text where the two
pre-tokenisers agree, and the decode(encode(s)) == s round trip.
"""

# tokenizer.c:332-343 -- bytes 33-126, 161-172, 174-255 keep their value as
# a code point, the other 68 bytes get 256, 257, ... in byte order.
def byte_alphabet():
    cps, nxt = [], 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            cps.append(b)
        else:
            cps.append(nxt)
            nxt += 1
    return cps


BYTE_CP = byte_alphabet()
CP_BYTE = {cp: b for b, cp in enumerate(BYTE_CP)}


# tokenizer.c:146-225 -- JSON string with \" \\ \/ \b \f \n \r \t and \uXXXX
# (a high surrogate followed by \uDC00-\uDFFF combines into one code point).
def _json_string(s, i):
    assert s[i] == '"'
    i += 1
    out = bytearray()
    while s[i] != '"':
        c = s[i]
        if c != "\\":
            out += c.encode("utf-8", "surrogatepass")
            i += 1
            continue
        e = s[i + 1]
        i += 2
        simple = {'"': '"', "\\": "\\", "/": "/", "b": "\b", "f": "\f", "n": "\n", "r": "\r", "t": "\t"}
        if e in simple:
            out += simple[e].encode()
            continue
        if e != "u":
            raise ValueError("bad escape")
        cp = int(s[i:i + 4], 16)
        i += 4
        if 0xD800 <= cp <= 0xDBFF and s[i:i + 2] == "\\u":
            lo = int(s[i + 2:i + 6], 16)
            if 0xDC00 <= lo <= 0xDFFF:
                cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00)
                i += 6
        out += _utf8(cp)
    return bytes(out), i + 1


def _utf8(cp):
    # tokenizer.c:33-45, surrogates included
    if cp < 0x80:
        return bytes([cp])
    if cp < 0x800:
        return bytes([0xC0 | (cp >> 6), 0x80 | (cp & 0x3F)])
    if cp < 0x10000:
        return bytes([0xE0 | (cp >> 12), 0x80 | ((cp >> 6) & 0x3F), 0x80 | (cp & 0x3F)])
    return bytes([0xF0 | (cp >> 18), 0x80 | ((cp >> 12) & 0x3F), 0x80 | ((cp >> 6) & 0x3F), 0x80 | (cp & 0x3F)])


class Tokenizer:
    def __init__(self, directory):
        self.vocab, self.id_str = {}, {}
        # tokenizer.c:227-283 -- "string": id pairs; a later duplicate wins
        text = open(f"{directory}/vocab.json", "rb").read().decode("utf-8", "surrogateescape")
        i = text.index("{") + 1
        while True:
            while text[i] in " \t\n\r,":
                i += 1
            if text[i] == "}":
                break
            key, i = _json_string(text, i)
            while text[i] in " \t":
                i += 1
            assert text[i] == ":"
            i += 1
            while text[i] in " \t":
                i += 1
            j = i
            while text[j].isdigit():
                j += 1
            val = int(text[i:j] or "0")
            i = j
            self.vocab[key] = val
            self.id_str[val] = key
        self.vocab_size = max(self.id_str) + 1 if self.id_str else 0
        # tokenizer.c:285-330 -- skip a '#' first line; "left right" lines
        # (first space), ranks in order, blank and space-less lines skipped
        raw = open(f"{directory}/merges.txt", "rb").read()
        lines = raw.split(b"\n")
        if raw.startswith(b"#"):
            lines = lines[1:]
        self.ranks, rank = {}, 0
        for ln in lines:
            ln = ln.rstrip(b"\r")
            if not ln or b" " not in ln:
                continue
            a, b = ln.split(b" ", 1)
            self.ranks[(a, b)] = rank
            rank += 1

    # tokenizer.c:360-421
    def _bpe(self, piece, out, max_ids):
        syms = [_utf8(BYTE_CP[b]) for b in piece]
        while len(syms) > 1:
            rs = [self.ranks.get((syms[k], syms[k + 1])) for k in range(len(syms) - 1)]
            cand = [r for r in rs if r is not None]
            if not cand:
                break
            best = min(cand)
            new, k = [], 0
            while k < len(syms):
                if k + 1 < len(syms) and self.ranks.get((syms[k], syms[k + 1])) == best:
                    new.append(syms[k] + syms[k + 1])
                    k += 2
                else:
                    new.append(syms[k])
                    k += 1
            syms = new
        for s in syms:
            if s in self.vocab and len(out) < max_ids:
                out.append(self.vocab[s])

    # tokenizer.c:423-550 -- ASCII classes; other = not space/letter/digit
    @staticmethod
    def pieces(data):
        def letter(c): return 65 <= c <= 90 or 97 <= c <= 122
        def digit(c): return 48 <= c <= 57
        def space(c): return c in b" \t\n\r\f\v"
        def same(c, k): return (not space(c)) and (letter(c) if k == 1 else digit(c) if k == 2
                                                   else not (letter(c) or digit(c)))
        def klass(c): return 1 if letter(c) else 2 if digit(c) else 3
        i, n = 0, len(data)
        while i < n:
            c = data[i]
            if c == 39 and i + 1 < n and data[i + 1] in b"stmd":
                j = i + 2
            elif c == 39 and i + 2 < n and data[i + 1:i + 3] in (b"re", b"ve", b"ll"):
                j = i + 3
            elif c == 32 and i + 1 < n and not space(data[i + 1]):
                k, j = klass(data[i + 1]), i + 2
                while j < n and same(data[j], k):
                    j += 1
            elif not space(c):
                k, j = klass(c), i + 1
                while j < n and same(data[j], k):
                    j += 1
            else:
                j = i + 1
            yield data[i:j]
            i = j

    def encode(self, text, max_ids=1023):
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        out = []
        for p in self.pieces(data):
            if len(out) >= max_ids:
                break
            self._bpe(p, out, max_ids)
        return out

    # tokenizer.c:552-579 -- code points back to bytes, '?' if unmapped; a
    # lead byte that is not UTF-8 ends the token; max_bytes - 1 bytes
    def decode(self, ids, max_bytes=1 << 30):
        out = bytearray()
        for t in ids:
            if t < 0 or t >= self.vocab_size or t not in self.id_str:
                continue
            s = self.id_str[t] + b"\0\0\0"
            j, end = 0, len(self.id_str[t])
            while j < end:
                c = s[j]
                if c < 0x80:
                    cp, u = c, 1
                elif c & 0xE0 == 0xC0:
                    cp, u = ((c & 0x1F) << 6) | (s[j + 1] & 0x3F), 2
                elif c & 0xF0 == 0xE0:
                    cp, u = ((c & 0x0F) << 12) | ((s[j + 1] & 0x3F) << 6) | (s[j + 2] & 0x3F), 3
                elif c & 0xF8 == 0xF0:
                    cp = ((c & 0x07) << 18) | ((s[j + 1] & 0x3F) << 12) | ((s[j + 2] & 0x3F) << 6) | (s[j + 3] & 0x3F)
                    u = 4
                else:
                    break
                if len(out) >= max_bytes - 1:
                    return bytes(out)
                out.append(CP_BYTE.get(cp, 63) if cp < 512 else 63)
                j += u
        return bytes(out)
