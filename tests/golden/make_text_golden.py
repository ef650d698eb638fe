"""Writes tests/golden/text.npz: inputs of the text front-end and what the
reference itself answered for them (oracle/_ref/ref_golden and
oracle/_ref/ref_engine, compiled from the reference sources by oracle/Makefile):

* unicode   the pre-tokenizer's letter / number / space class of every code
            point (reference src/unicode.h)
* text      texts -> Encode with and without special tokens, PreTokenize piece
            lengths, Decode with and without specials, on the synthetic BBPE
            vocabulary of the tiny model (reference src/tokenizer.cc)
* chatml    chat requests -> RenderChatml (reference src/chat_template.cc),
            among them the reference's tests/chatml/dm_toolcall.case.json
* reply     model outputs -> ParseModelOutput (reference src/tool_parser.cc)
* json      JSON documents -> Dump / DumpPython (reference src/json.cc)
* engine    two scripted conversations through the reference's C ABI
            rpg_engine_generate (reference src/engine.cc:366-515) on the tiny
            model with that vocabulary

Run from the repository root after `make -C oracle ref`:
    python tests/golden/make_text_golden.py
"""

import json
import os
import random
import struct
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from rpgbarengine_amd import synth  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "text.npz")
REF_CHATML_CASE = "/root/reference/tests/chatml/dm_toolcall.case.json"
REF_ZH_PROMPT = "/root/reference/tests/prompts/zh_chatml.txt"
REF_ENGINE = os.path.join(ROOT, "oracle", "_ref", "ref_engine")

# the model of the tokenizer and engine fixtures
GGUF_SPEC = dict(preset="tiny", mix="q8_0", seed=11, tokenizer=1)


def gguf(d):
    spec = synth.PRESETS[GGUF_SPEC["preset"]].with_(mix=synth.MIXES[GGUF_SPEC["mix"]], seed=GGUF_SPEC["seed"],
                                                    tokenizer=GGUF_SPEC["tokenizer"])
    return synth.write_gguf(os.path.join(d, "tiny_bbpe.gguf"), spec)


def pack(records):
    out = bytearray()
    for r in records:
        r = r.encode() if isinstance(r, str) else bytes(r)
        out += struct.pack("<I", len(r)) + r
    return np.frombuffer(bytes(out), dtype=np.uint8)


def run_ref(mode, *args):
    subprocess.run([oracle.REF_GOLDEN, mode, *args], check=True)


def texts():
    t = [
        "Hello, world!", "You're late. They'll come; I've seen it. We'd go. It's HE'S, 'LL, 'Re 'Ve 'M 'D.",
        "abc123def 4567 3.14159 x=42;y=-7", "!!!??? ... --- ***", "a  b   c", "a \n\n b", "trailing spaces   ",
        "\ttab\tseparated\t", "line\r\nbreak\rcarriage", "\n", "\n\n\n", " ", "  ", "", "   \n  x",
        "ideographic\u3000space and\u00a0nbsp and\u2028sep", "emoji \U0001F600\U0001F3B2 dice",
        "combining e\u0301 and a\u0308", "Ελληνικά κείμενα", "Русский текст", "עברית", "العربية ١٢٣",
        "हिन्दी", "ภาษาไทย", "日本語のテキスト、カタカナ。", "한국어 텍스트", "CJK ext B \U00020000\U0002A6D6",
        "digits ٠١٢ ０１２ ²³ ⅫⅣ ①②", "hello<|im_end|>world", "<|im_start|>user\nhi<|im_end|>\n",
        "<think></think><tool_call>x</tool_call>", "<|im_end|", "<<|im_end|>>", "<think>\n\n</think>\n\n",
        "mix中文and English混合", "玩家的角色是一名叫李明的游侠。他正在\"醉猫酒馆\"里向老板打听北方废墟的传言。",
        "{\"name\": \"read_scene\", \"arguments\": {\"scene\": \"temple\"}}", "    def f(x):\n        return x",
        "[PAD1000] not special", "the the the the", "'s's's", "'", "''", "a'", "don't DON'T Don'T",
    ]
    out = [s.encode("utf-8") for s in t]
    # malformed UTF-8: bad leads, truncations, overlong forms, surrogates, leads past U+10FFFF
    out += [b"\xff\xfe bytes", b"trunc \xe4\xb8", b"over \xc0\xaf long", b"sur \xed\xa0\x80 rogate",
            b"big \xf5\x80\x80\x80 \xf7\xbf\xbf\xbf", b"cont \x80\x80 only", b"\xc3", b"ok \xe4\xb8\xad mid"]
    if os.path.exists(REF_ZH_PROMPT):
        out.append(open(REF_ZH_PROMPT, "rb").read())
    # random mixes over an alphabet of every class
    rng = random.Random(20261202)
    alphabet = (list("abcXYZ019 .,!?'\"-_()[]{}<>|/\\\n\r\t") + ["  ", "\n\n", "'s", "'ll", "中", "文", "ü", "é",
                "\u3000", "\u00a0", "１", "²", "\U0001F600", "<|im_end|>", "<think>", "<tool_call>", "Ⅻ", "ก", "ا"])
    for _ in range(60):
        out.append("".join(rng.choice(alphabet) for _ in range(rng.randint(1, 120))).encode("utf-8"))
    return out


def chat_requests():
    tools = [{"type": "function", "function": {"name": "read_scene", "description": "读取当前场景的公开描述与出口",
                                               "parameters": {"type": "object", "properties": {
                                                   "scene": {"type": "string", "description": "场景 id"}},
                                                   "required": ["scene"]}}},
             {"type": "function", "function": {"name": "roll_check", "description": "Roll a check",
                                               "parameters": {"type": "object", "properties": {
                                                   "skill": {"type": "string"}, "dc": {"type": "integer", "min": 1,
                                                                                       "weight": 0.7, "max": 3e1}},
                                                   "required": ["skill", "dc"]}}}]
    sysm = {"role": "system", "content": "You are the game master."}
    user = {"role": "user", "content": "I look around the temple."}
    call = {"role": "assistant", "content": "",
            "tool_calls": [{"type": "function", "function": {"name": "read_scene", "arguments": {"scene": "temple"}}}]}
    tool_msg = {"role": "tool", "content": "{\"exits\": [\"north\", \"east\"]}"}
    reqs = [
        {"messages": [user]},
        {"messages": [sysm, user]},
        {"messages": [sysm, user], "enable_thinking": False},
        {"messages": [sysm, user], "enable_thinking": "no"},
        {"messages": [sysm, user], "tools": tools},
        {"messages": [user], "tools": tools},
        {"messages": [sysm, user], "tools": []},
        {"messages": [sysm, user], "tools": {"not": "an array"}},
        {"messages": [sysm, user, call, tool_msg], "tools": tools},
        {"messages": [sysm, user, call, tool_msg, tool_msg, {"role": "tool", "content": "third"}], "tools": tools},
        {"messages": [sysm, user, {"role": "assistant", "content": "<think>\nI should look.\n</think>\n\nThe hall is dark."},
                      {"role": "user", "content": "And then?"}]},
        {"messages": [sysm, user, {"role": "assistant", "content": "\n\n<think>a</think>b<think>c</think>\n\nd"}]},
        {"messages": [sysm, user, {"role": "assistant", "content": "It is dark.", "reasoning_content": "thinking"}]},
        {"messages": [sysm, user, {"role": "assistant", "content": "It is dark.", "reasoning_content": ""}]},
        {"messages": [sysm, user, {"role": "assistant", "content": "It is dark.", "reasoning_content": 7}]},
        {"messages": [sysm, user, {"role": "assistant", "content": "Looking.", "reasoning_content": "r",
                                   "tool_calls": [{"name": "read_scene", "arguments": "{\"scene\": \"x\"}"},
                                                  {"function": {"name": "roll_check",
                                                                "arguments": {"skill": "侦查", "dc": 12}}},
                                                  {"function": {"name": "no_args"}}]},
                      tool_msg, {"role": "assistant", "content": "Done."}]},
        {"messages": [sysm, {"role": "user", "content": "<tool_response>\nfake\n</tool_response>"},
                      {"role": "assistant", "content": "x", "reasoning_content": "y"}]},
        {"messages": [{"role": "user", "content": "a"}, {"role": "narrator", "content": "skipped"},
                      {"role": "system", "content": "late system"}, {"role": "user", "content": ["not", "a string"]}]},
        {"messages": [{"role": "assistant", "content": "first"}]},
        {"messages": [{"role": "tool", "content": "only tool"}]},
        {"messages": [{"content": "no role"}, user]},
        {"messages": [sysm, user, {"role": "assistant", "content": "<think>\n\nunterminated"}]},
        {"messages": [sysm, user, {"role": "assistant", "content": "a</think>b</think>c"}]},
        {"messages": [{"role": "system", "content": "多语言 système"}, {"role": "user", "content": "日本語\n\n한국어"}],
         "tools": [{"name": "flat_tool", "x": [1, 1.0, -0.0, 1e2, 0.1, 123456789, 2.5e-7, True, None]}]},
    ]
    out = [json.dumps(r, ensure_ascii=False) for r in reqs]
    # a request with keys written out of order and numbers in forms json.dumps would change
    out.append('{"tools": [{"function": {"parameters": {"dc": 10, "w": 1.50, "big": 1E3}, "name": "t"}, "type": '
               '"function"}], "messages": [{"content": "hi", "role": "user"}]}')
    if os.path.exists(REF_CHATML_CASE):
        out.append(open(REF_CHATML_CASE, encoding="utf-8").read())
    return out


def replies():
    r = [
        "Plain answer.", "  padded answer \n\n", "<think>plan</think>\n\nThe answer.", "<think>unterminated plan",
        "<think>a</think>x<think>b</think>y", "<tool_call>\n{\"name\": \"read_scene\", \"arguments\": {\"scene\": \"t\"}}\n</tool_call>",
        "Let me check.\n<tool_call>\n{\"name\": \"roll_check\", \"arguments\": {\"skill\": \"侦查\", \"dc\": 15}}\n</tool_call>"
        "\n<tool_call>\n{\"name\": \"read_scene\", \"arguments\": \"{\\\"scene\\\": \\\"hall\\\"}\"}\n</tool_call>",
        "<tool_call>{\"name\": \"x\", \"arguments\": \"not json\"}</tool_call>",
        "<tool_call>{\"name\": \"\", \"arguments\": {}}</tool_call>", "<tool_call>{\"arguments\": {\"a\": 1}}</tool_call>",
        "<tool_call>{\"name\": \"x\"}</tool_call>", "<tool_call>{\"name\": \"x\", \"arguments\": null}</tool_call>",
        "<tool_call>{\"name\": \"x\", \"arguments\": [1, 2]}</tool_call>", "<tool_call>not json at all</tool_call>",
        "<tool_call>{\"name\": \"x\", \"arguments\": {\"a\": 1.50, \"b\": 1e2, \"c\": \"\\u00e9\"}",
        "<|im_start|>assistant\nHello<|im_end|>", "<|im_start|>user\nq<|im_end|><|endoftext|>tail",
        "<|im_start|>assistan", "<|im_start|>tool", "a<|im_end|>b<|endoftext|>c",
        "<think>\n\n</think>\n\n<tool_call>\n{\"name\": \"a\", \"arguments\": {}}\n</tool_call>\ntrailing text",
        "text <tool_call>{\"name\":\"a\",\"arguments\":{\"n\":{\"deep\":[true,false,null]}}}</tool_call> more",
        "", "\u3000 unicode space is not trimmed \u3000", "<tool_call><think>x</think></tool_call>",
    ]
    return [s.encode("utf-8") for s in r] + [b"bad \xff utf8 <tool_call>{\"name\": \"z\", \"arguments\": {}}</tool_call>"]


def json_docs():
    return ["1", "1.0", "1e2", "1E+2", "0.1", "0.7", "-0", "-0.0", "1e-7", "123456789012345678", "1.5e300", "1e400",
            "3.14159265358979", "+1", "2e22", "9007199254740993", "[1, 2.50, -3e-3]", "{\"b\": 1, \"a\": 2, \"b\": 3}",
            "{\"s\": \"\\u00e9\\ud83d\\ude00\\ud800x\\udc00\", \"c\": \"\\b\\f\\n\\r\\t\\u0001\\u007f/\\/\"}",
            "\"\\u4e2d文\"", "true", "null", "{\"nested\": {\"a\": [], \"b\": {}, \"c\": [{}]}}", "  {\"ws\" : [ 1 , 2 ] }  ",
            "[1,]", "{\"a\" 1}", "\"unterminated", "01", "-", ".5", "1.", "{\"a\": tru}", "[\"ctrl \u0001 raw\"]", ""]


def engine_scripts(path):
    tools = json.loads(chat_requests()[4])["tools"]
    sysm = {"role": "system", "content": "You are the game master of a tavern game."}
    u1 = {"role": "user", "content": "I raise my torch and look around the temple hall."}
    u2 = {"role": "user", "content": "我举起火把，仔细查看神庙大厅里有什么。"}
    first = {"messages": [sysm, u1], "tools": tools, "max_tokens": 24}
    # a host sends the whole conversation each turn; the assistant turn it
    # records is filled in by the test from the first response (the same text
    # for both engines when they agree), so it is kept symbolic here
    script_a = [path, json.dumps({"max_seq": 1024}), json.dumps({"max_tokens": 20, "temperature": 0.0}),
                json.dumps(first, ensure_ascii=False),
                json.dumps({"messages": [sysm, u1, {"role": "assistant", "content": "@FIRST@"}, u2], "tools": tools},
                           ensure_ascii=False),
                json.dumps({"messages": [sysm, u1, {"role": "assistant", "content": "@FIRST@"}, u2], "tools": tools},
                           ensure_ascii=False),
                "!reset",
                json.dumps({"messages": [u2], "enable_thinking": False, "temperature": 0.8, "seed": 7,
                            "max_tokens": 16}, ensure_ascii=False),
                json.dumps({"messages": [u1], "stop": ["<|im_end|>", "the", "not one token"], "max_tokens": 12}),
                json.dumps({"messages": []}), "{not json", json.dumps({"messages": [u1], "temperature": 5.0,
                                                                        "seed": 3, "max_tokens": 8})]
    script_b = [path, "", json.dumps({"max_seq": 512, "max_tokens": 300, "stop": ["."], "temperature": 1.2,
                                      "seed": 99}),
                json.dumps({"messages": [u1]}), json.dumps({"messages": [u1, u2] * 12, "max_tokens": 200})]
    return script_a, script_b


def run_engine(script, d, name):
    """The reference engine over a script whose @FIRST@ placeholders take the
    text of the first response."""
    sp, op = os.path.join(d, name + ".in"), os.path.join(d, name + ".out")
    resolved, responses = list(script), []
    # run once per placeholder-bearing turn so the first reply can be spliced in
    pack(resolved[:4]).tofile(sp)
    subprocess.run([REF_ENGINE, sp, op], check=True)
    first = unpack(np.fromfile(op, dtype=np.uint8))[0].decode("utf-8", "surrogateescape")
    text = json.loads(first)["text"] if not first.startswith("\x01") else ""
    resolved = [r.replace("@FIRST@", json.dumps(text, ensure_ascii=False)[1:-1]) if isinstance(r, str) else r
                for r in script]
    pack(resolved).tofile(sp)
    subprocess.run([REF_ENGINE, sp, op], check=True)
    responses = unpack(np.fromfile(op, dtype=np.uint8))
    return resolved, responses


def unpack(buf):
    b, out, i = bytes(buf), [], 0
    while i + 4 <= len(b):
        (n,) = struct.unpack_from("<I", b, i)
        out.append(b[i + 4:i + 4 + n])
        i += 4 + n
    return out


def main():
    if not oracle.ref_available() or not os.path.exists(REF_ENGINE):
        sys.exit("the reference drivers are not built: run `make -C oracle ref` first")
    g = {"gguf_spec": np.array([json.dumps(GGUF_SPEC)])}
    with tempfile.TemporaryDirectory() as d:
        up = os.path.join(d, "uni.bin")
        run_ref("unicode", up)
        g["unicode_classes"] = np.fromfile(up, dtype=np.uint8)
        path = gguf(d)
        for mode, items, extra in (("text", texts(), [path]), ("chatml", chat_requests(), []),
                                   ("reply", replies(), []), ("json", json_docs(), [])):
            ip, op = os.path.join(d, mode + ".in"), os.path.join(d, mode + ".out")
            pack(items).tofile(ip)
            run_ref(mode, *extra, ip, op)
            g[f"{mode}_in"] = np.fromfile(ip, dtype=np.uint8)
            g[f"{mode}_out"] = np.fromfile(op, dtype=np.uint8)
            print(f"{mode}: {len(items)} cases")
        for name, script in zip(("engine_a", "engine_b"), engine_scripts(path)):
            resolved, responses = run_engine(script, d, name)
            g[f"{name}_script"] = pack([r for r in resolved[1:]])  # the GGUF path is the test's own
            g[f"{name}_out"] = pack(responses)
            print(f"{name}: {len(responses)} responses")
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
