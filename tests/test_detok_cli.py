"""Host checks of the text side that need no GPU: the byte-level BPE detokenizer
(src/detok.h:13-41) against GPT-2's published bytes_to_unicode map, written out here
independently, and the CLI's argument errors (cpu_infer.cpp:64-68: usage on stderr,
exit status 1) which return before any device call."""
import os
import subprocess

import minfer

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "nano-inference_amd", "_build", "minfer")


def bytes_to_unicode():
    """GPT-2 encoder.py: printable bytes keep their code point, the rest get 256 + n"""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAC + 1)) + list(range(0xAE, 0xFF + 1))
    cs = bs[:]
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return dict(zip(bs, (chr(c) for c in cs)))


def test_detok_every_byte_round_trips():
    enc = bytes_to_unicode()
    assert len(enc) == 256 and max(ord(c) for c in enc.values()) == 323
    for b in range(256):
        assert minfer.detok_piece(enc[b]) == bytes([b]), b
    everything = "".join(enc[b] for b in range(256))
    assert minfer.detok_piece(everything) == bytes(range(256))


def test_detok_known_pieces():
    assert minfer.detok_piece("Ġhello") == b" hello"          # 'Ġ' = byte 0x20
    assert minfer.detok_piece("ĊĊ") == b"\n\n"            # 'Ċ' = byte 0x0A
    assert minfer.detok_piece("<|im_end|>") == b"<|im_end|>"
    # UTF-8 text in pieces is stored byte by byte: "é" = C3 A9 -> code points Ã (0xC3), © (0xA9)
    assert minfer.detok_piece("Ã©") == "é".encode()
    # code points outside the map are dropped, as are malformed lead bytes
    assert minfer.detok_piece("a中b") == b"ab"
    assert minfer.detok_piece(b"a\xffb") == b"ab"
    assert minfer.detok_piece(b"") == b""


def test_detok_reports_full_length_past_cap():
    import ctypes as C
    buf = C.create_string_buffer(4)
    n = minfer.lib().mi_detok_piece(b"abcdefgh", 8, buf, 4)
    assert n == 8 and buf.raw[:4] == b"abcd"
    assert minfer.lib().mi_detok_piece(None, 3, buf, 4) == -1


def test_cli_usage_and_bad_arguments():
    assert os.path.exists(CLI), "CLI not built"
    r = subprocess.run([CLI], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "usage:" in r.stderr and r.stdout == ""
    r = subprocess.run([CLI, "x.gguf", "-3", "1"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "n_gen" in r.stderr
