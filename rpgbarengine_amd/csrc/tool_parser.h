// Parse of a generated reply (decoded with its special tokens kept) into
// the text for the host, the reasoning and the tool calls, the behaviour of
// the reference's output parser (reference src/tool_parser.h:1-69,
// src/tool_parser.cc):
//   1. control markers go: every <|im_start|> (with a following
//      "system\n" / "user\n" / "assistant\n" / "tool\n"), <|im_end|> and
//      <|endoftext|>;
//   2. <think> ... </think> blocks are cut out (their bodies concatenated
//      into the reasoning); an unclosed <think> takes the rest of the text;
//   3. <tool_call> ... </tool_call> blocks become calls and are cut out; an
//      unclosed one is still parsed from what is there;
//   4. the remaining text is trimmed of ASCII whitespace.
// A call body is JSON {"name": ..., "arguments": ...}; a string argument
// holding a JSON object is unwrapped; a call is usable when it has a name and
// an object of arguments.

#ifndef RPG_HIP_TOOL_PARSER_H_
#define RPG_HIP_TOOL_PARSER_H_

#include <string>
#include <vector>

#include "json_min.h"

namespace rpg {

struct ParsedCall {
  std::string name;
  std::string arguments_raw;  // the arguments as written (logged when unusable)
  JValue arguments;           // null unless an object
  bool ok = false;
};

struct ParsedReply {
  std::string text, reasoning;
  std::vector<ParsedCall> calls;
  bool unterminated_think = false, unterminated_call = false;
};

ParsedReply ParseReply(const std::string& raw);

}  // namespace rpg

#endif  // RPG_HIP_TOOL_PARSER_H_
