// Test harness for the pack reader built with AddressSanitizer (host code
// only): opens every file named on the command line with uqm_pack_open, looks
// up each tensor named in the file's header, reads every byte of it, closes.
// Prints one line per file: "ok <tensors>" or "refused <code> <message>".
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../include/uma_qmoe_pack.h"

// The library's error plumbing (uqm_api.hip), restated for this host-only build.
static thread_local std::string g_error;
namespace uqm {
int api_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}
}  // namespace uqm
extern "C" const char* uqm_last_error(void) { return g_error.c_str(); }

namespace {
// A minimal scan for "name":"..." entries of the header (test input only).
std::vector<std::string> tensor_names(const char* json, size_t n) {
  std::vector<std::string> out;
  const std::string s(json, n);
  const std::string key = "\"name\":\"";
  for (size_t p = s.find(key); p != std::string::npos; p = s.find(key, p + 1)) {
    const size_t a = p + key.size(), b = s.find('"', a);
    if (b == std::string::npos) break;
    out.push_back(s.substr(a, b - a));
  }
  return out;
}
}  // namespace

int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i) {
    uqm_pack* pack = nullptr;
    const int rc = uqm_pack_open(argv[i], UQM_PACK_ANY, nullptr, nullptr, nullptr, nullptr, &pack);
    if (rc != 0) {
      printf("refused %d %s\n", rc, uqm_last_error());
      continue;
    }
    const char* json = nullptr;
    size_t n = 0;
    if (uqm_pack_header(pack, &json, &n) != 0) return 2;
    unsigned sum = 0;
    int count = 0;
    for (const std::string& name : tensor_names(json, n)) {
      uqm_pack_tensor t;
      if (uqm_pack_lookup(pack, name.c_str(), &t) != 0) continue;
      for (uint64_t k = 0; k < t.data_bytes; ++k) sum += t.data[k];
      for (uint64_t k = 0; k < t.scale_bytes; ++k) sum += t.scales[k];
      ++count;
    }
    int32_t enc = -1;
    (void)uqm_pack_layer_encoding(pack, 0, &enc);
    (void)uqm_pack_layer_encoding(pack, 1000, &enc);
    uqm_pack_close(pack);
    printf("ok %d %u\n", count, sum & 1u);
  }
  return 0;
}
