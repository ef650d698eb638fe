// Qwen3 ChatML rendering of a chat request: messages (+ tools) -> prompt
// text, the behaviour of the official Qwen3 chat template as the reference
// renders it (reference src/chat_template.h:1-81, src/chat_template.cc).
//
//   * with tools, one system block: the first system message's content (if
//     any) + "\n\n", the tools preamble, one line per tool (json.dumps style:
//     ", " / ": ", non-ASCII kept), the tool-call instructions;
//     without tools, the first system message as its own block;
//   * user messages, and system messages after the first, as plain blocks;
//   * an assistant message's reasoning is its reasoning_content when that
//     is a string, else what its content holds between <think> and the
//     first </think>; the think block is rendered only after the last real
//     user query (a user message not wholly wrapped in <tool_response>
//     tags) and only for the last message or a message with reasoning;
//     its tool calls follow as <tool_call> blocks;
//   * consecutive tool messages share one user block, each wrapped in
//     <tool_response> tags;
//   * unknown roles are skipped; the generation prompt opens an assistant
//     block, with an empty think block when enable_thinking is false.
// Only '\n' is stripped where the template strips (Python's strip('\n')).

#ifndef RPG_HIP_CHATML_H_
#define RPG_HIP_CHATML_H_

#include <string>
#include <vector>

#include "json_min.h"

namespace rpg {

struct ChatToolCall {
  std::string name;
  std::string arguments = "{}";  // JSON text, written into the prompt as it is
};

struct ChatMessage {
  std::string role, content;
  bool has_reasoning = false;  // reasoning_content given as a string (even empty)
  std::string reasoning;
  std::vector<ChatToolCall> tool_calls;
};

// Lenient reading of a request's "messages": missing or mistyped fields take
// the template's defaults (content "", no tool calls); a tool call may be
// {"function": {...}} or flat; object arguments are dumped json.dumps style.
std::vector<ChatMessage> ParseChatMessages(const JValue& messages);

// "tools" when it is an array, else an empty array (the no-tools branch).
JValue ParseChatTools(const JValue& tools);

std::string RenderChatml(const std::vector<ChatMessage>& messages, const JValue& tools,
                         bool add_generation_prompt, bool enable_thinking);

}  // namespace rpg

#endif  // RPG_HIP_CHATML_H_
