// qdiy_engine: the reference engine's command-line sidecar on MI355X
// (framework_src/qwen_infer.cu:743-822), driven by web_chat/app.py over
// stdin/stdout (app.py:63-85, 214-251).
//
//   qdiy_engine [--prefill exact|mfma] [model.bin]
//                                    model default ../model_weights/qwen_1.8b.bin
//
// --prefill (or the environment variable QDIY_PREFILL when the flag is absent)
// picks how prompts are prefilled: "exact" (the default) leaves the KV cache
// bit-identical to decoding the prompt token by token; "mfma" runs the
// projections and the causal attention on the matrix cores, as the
// reference's prefill runs them on tensor cores (qwen_infer.cu:791-794 ->
// :372-611), ~17x faster on a 2048-token prompt, but its rounding differs,
// so tokens after a prompt can differ at near-ties.
//
// Protocol, one request per stdin line:
//   "exit" or an empty line          ends the process
//   "reset"                          clears the KV cache, answers [RESET_DONE]
//   "t0 t1 ... tn"                   space-separated prompt token ids:
//                                    [GENERATION_START], then one generated id
//                                    per line (at most 512, stopping before
//                                    151645 / 151643), then [GENERATION_END]
// After loading, the process prints a line containing [ENGINE_READY].
#include <cstdlib>
#include <iostream>
#include <string>
#include <vector>

#include "qdiy/decode.h"
#include "qdiy/engine.h"

namespace {

constexpr int kMaxNewTokens = 512;   // qwen_infer.cu:797

// Splits on single spaces as the reference does (qwen_infer.cu:770-784);
// returns false on a token that is not a decimal integer.
bool parse_tokens(const std::string& line, std::vector<int>& out) {
  std::string cur;
  auto flush = [&]() {
    if (cur.empty()) return true;
    size_t used = 0;
    try {
      const long v = std::stol(cur, &used);
      if (used != cur.size() || v < -2147483648L || v > 2147483647L) return false;
      out.push_back((int)v);
    } catch (...) {
      return false;
    }
    cur.clear();
    return true;
  };
  for (char c : line) {
    if (c == ' ') {
      if (!flush()) return false;
    } else {
      cur += c;
    }
  }
  return flush();
}

}  // namespace

int main(int argc, char** argv) {
  std::cout << std::unitbuf;
  std::string path = "../model_weights/qwen_1.8b.bin";
  const char* env_mode = std::getenv("QDIY_PREFILL");
  std::string mode = env_mode ? env_mode : "exact";
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--prefill" && i + 1 < argc) {
      mode = argv[++i];
    } else if (a.rfind("--prefill=", 0) == 0) {
      mode = a.substr(10);
    } else if (!a.empty() && a[0] == '-') {
      std::cerr << "Error: unknown option " << a << " (usage: qdiy_engine [--prefill exact|mfma] [model.bin])"
                << std::endl;
      return 2;
    } else {
      path = a;
    }
  }
  if (mode != "exact" && mode != "mfma") {
    std::cerr << "Error: prefill mode must be exact or mfma, got " << mode << std::endl;
    return 2;
  }
  qd_engine* eng = nullptr;
  if (qd_engine_create(path.c_str(), &eng) != QD_OK) {
    std::cerr << "Error: " << qd_last_error() << std::endl;
    return 1;
  }
  if (mode == "mfma" && qd_engine_set_prefill_mode(eng, QD_GEMM_MFMA) != QD_OK) {
    std::cerr << "Error: " << qd_last_error() << std::endl;
    qd_engine_destroy(eng);
    return 1;
  }
  qd_model_cfg c;
  qd_engine_config(eng, &c);
  std::cout << "\n=== Weight Config Loaded ===\n  Vocab size:        " << c.vocab_size
            << "\n  Hidden size:       " << c.hidden_size << "\n  Layers count:      " << c.num_layers
            << "\n  Heads count:       " << c.num_heads << "\n  FFN Intermediate:  " << c.intermediate_size
            << "\n  Max seqlen:        " << c.max_seqlen << "\n  Prefill:           " << mode
            << std::endl;
  std::cout << "\n[ENGINE_READY] MI355X (gfx950) Qwen inference engine is fully ready." << std::endl;

  std::string line;
  while (std::getline(std::cin, line)) {
    if (!line.empty() && line.back() == '\r') line.pop_back();
    if (line.empty() || line == "exit") break;
    if (line == "reset") {
      if (qd_engine_reset(eng) != QD_OK) std::cerr << "[ERROR] reset: " << qd_last_error() << std::endl;
      std::cout << "[RESET_DONE]" << std::endl;
      continue;
    }
    std::vector<int> prompt;
    if (!parse_tokens(line, prompt)) {
      std::cerr << "[ERROR] cannot parse token ids: " << line << std::endl;
      continue;
    }
    if (prompt.empty()) continue;
    int pos = 0;
    bool ok = true;
    if (prompt.size() > 1 && qd_engine_prefill(eng, prompt.data(), (int)prompt.size() - 1, &pos) != QD_OK) {
      std::cerr << "[ERROR] prefill: " << qd_last_error() << std::endl;
      ok = false;
    }
    int last = prompt.back();
    std::cout << "[GENERATION_START]" << std::endl;
    for (int i = 0; ok && i < kMaxNewTokens; ++i) {
      int next = 0;
      if (qd_engine_step(eng, last, pos, &next) != QD_OK) {
        std::cerr << "[ERROR] step at position " << pos << ": " << qd_last_error() << std::endl;
        break;
      }
      ++pos;
      if (next == 151645 || next == 151643) break;   // ChatML stop tokens (qwen_infer.cu:801)
      std::cout << next << std::endl;
      last = next;
    }
    std::cout << "[GENERATION_END]" << std::endl;
  }
  qd_engine_destroy(eng);
  return 0;
}
