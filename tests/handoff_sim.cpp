// Host-side checks of the record-stream GEMM's hand-off protocol, built by
// tests/test_handoff_cpu.py with g++ against moat_amd/csrc/handoff.h (the
// same functions the kernel calls).  Prints one "ok <name>" line per check
// and exits nonzero at the first failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "handoff.h"

using namespace moat;

static int fails = 0;
#define CHECK(c)                                                    \
  do {                                                              \
    if (!(c)) {                                                     \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);      \
      ++fails;                                                      \
      return;                                                       \
    }                                                               \
  } while (0)

static uint32_t fbits(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return b;
}

// Every fp32 bit pattern: the encoding is never 0 ("not written"), decodes
// back to the same bits for every non-NaN value and to the canonical NaN for
// every NaN.
static void encoding_exhaustive() {
  uint64_t nans = 0;
  for (uint64_t i = 0; i <= 0xFFFFFFFFull; ++i) {
    const uint32_t b = (uint32_t)i;
    const uint32_t w = handoff_encode(b);
    if (w == 0u) CHECK(!"a value encodes to the empty word");
    const uint32_t d = handoff_decode(w);
    if (handoff_is_nan(b)) {
      ++nans;
      if (d != 0x7FC00000u) CHECK(!"NaN does not decode to the canonical NaN");
    } else if (d != b) {
      CHECK(!"value does not round-trip");
    }
  }
  CHECK(nans == 2ull * ((1ull << 23) - 1));  // both signs, every nonzero mantissa
  CHECK(!handoff_is_nan(fbits(INFINITY)) && !handoff_is_nan(fbits(-INFINITY)));
  CHECK(handoff_is_nan(fbits(NAN)));
  std::printf("ok encoding_exhaustive\n");
}

static void chunk_rules() {
  CHECK(handoff_chunk_written(1, 2, 3, 4));
  CHECK(!handoff_chunk_written(0, 2, 3, 4) && !handoff_chunk_written(1, 2, 3, 0));
  CHECK(handoff_stop(true, 5) && !handoff_gave_up(true, 5));
  CHECK(!handoff_stop(false, 5));
  CHECK(handoff_stop(false, 0) && handoff_gave_up(false, 0));
  CHECK(handoff_stop(true, 0) && !handoff_gave_up(true, 0));
  std::printf("ok chunk_rules\n");
}

// A simulated workspace: `slots` chunks of four words and a status word,
// used by calls of a tile group with `contrib` contributors.  The owner
// follows the kernel's gather: poll the contributors' chunks, stop when all
// are written or the budget is gone, add the decoded words, set the status
// on a give-up, clear every chunk of the batch, and write NaN when the
// status was already set at the start of the call.
struct Workspace {
  uint32_t status = 0;
  std::vector<uint32_t> words;
  explicit Workspace(int chunks) : words(4 * chunks, 0u) {}
};

struct Call {
  std::vector<float> partial;     // contributor c's value (the same in its four words)
  std::vector<int> store_at;      // poll count at which contributor c's store lands (-1: before the owner);
                                  // kBeforeClear: after the owner's last poll, before its clear
};
constexpr int kBeforeClear = 1 << 30;

// Returns the owner's four sums.
static std::vector<float> run_call(Workspace& ws, const Call& call, int budget, float own) {
  const uint32_t status0 = ws.status;
  const int contrib = (int)call.partial.size();
  auto land = [&](int c) {
    for (int e = 0; e < 4; ++e) ws.words[4 * c + e] = handoff_encode(fbits(call.partial[c]));
  };
  for (int c = 0; c < contrib; ++c)
    if (call.store_at[c] < 0) land(c);
  int polls = budget, polled = 0;
  std::vector<uint32_t> seen(4 * contrib);
  bool all;
  for (;;) {
    for (int c = 0; c < contrib; ++c)
      if (call.store_at[c] == polled) land(c);
    for (int i = 0; i < 4 * contrib; ++i) seen[i] = ws.words[i];
    all = true;
    for (int c = 0; c < contrib; ++c)
      all = all && handoff_chunk_written(seen[4 * c], seen[4 * c + 1], seen[4 * c + 2], seen[4 * c + 3]);
    if (handoff_stop(all, polls)) break;
    --polls;
    ++polled;
  }
  if (handoff_gave_up(all, polls)) ws.status |= kWsStatusHandoffTimeout;
  std::vector<float> out(4, 0.0f);
  for (int c = 0; c < contrib; ++c)
    for (int e = 0; e < 4; ++e) {
      uint32_t d = handoff_decode(seen[4 * c + e]);
      float f;
      std::memcpy(&f, &d, 4);
      out[e] += f;
    }
  for (int c = 0; c < contrib; ++c)
    if (call.store_at[c] == kBeforeClear) land(c);
  for (int c = 0; c < contrib; ++c)  // the owner clears every chunk of the batch
    for (int e = 0; e < 4; ++e) ws.words[4 * c + e] = 0u;
  for (int e = 0; e < 4; ++e) out[e] = status0 ? NAN : out[e] + own;
  // stores that land after the owner's clear
  for (int c = 0; c < contrib; ++c)
    if (call.store_at[c] > polled && call.store_at[c] != kBeforeClear) land(c);
  return out;
}

static bool all_zero(const Workspace& ws) {
  for (uint32_t w : ws.words)
    if (w) return false;
  return true;
}

static void protocol() {
  Workspace ws(3);
  // every partial there, some late but within the budget: exact sums, the
  // workspace left at zero, no status
  Call a{{1.5f, -2.0f, 0.25f}, {-1, 3, 7}};
  std::vector<float> r = run_call(ws, a, 100, 10.0f);
  CHECK(r[0] == 9.75f && r[3] == 9.75f);
  CHECK(all_zero(ws) && ws.status == 0);
  // a negative zero and an infinity travel intact
  Call b{{-0.0f, INFINITY, 1.0f}, {-1, -1, -1}};
  r = run_call(ws, b, 4, 0.0f);
  CHECK(std::isinf(r[0]) && r[0] > 0 && all_zero(ws));
  // a NaN partial is a written value, not "missing"
  Call c{{NAN, 1.0f, 2.0f}, {-1, -1, 0}};
  r = run_call(ws, c, 4, 0.0f);
  CHECK(std::isnan(r[0]) && all_zero(ws) && ws.status == 0);
  // contributor 1 stores after the budget runs out: NaN for this call, the
  // status set, the other chunks cleared, and the late chunk left behind
  Call d{{1.0f, 2.0f, 3.0f}, {-1, 50, -1}};
  r = run_call(ws, d, 8, 0.0f);
  CHECK(std::isnan(r[0]) && ws.status == kWsStatusHandoffTimeout);
  CHECK(ws.words[0] == 0 && ws.words[8] == 0 && ws.words[4] != 0);  // the chunk that landed after the clear
  // the next call finds the stale chunk and would add it as its own; the
  // status turns its results into NaN instead of silently wrong values
  Call e{{4.0f, 5.0f, 6.0f}, {-1, 2, -1}};
  r = run_call(ws, e, 8, 0.0f);
  CHECK(std::isnan(r[0]) && std::isnan(r[3]));
  // a late store that lands before the owner's clear is removed by it
  ws = Workspace(3);
  Call f{{1.0f, 2.0f, 3.0f}, {-1, kBeforeClear, -1}};
  r = run_call(ws, f, 8, 0.0f);
  CHECK(std::isnan(r[0]) && ws.status == kWsStatusHandoffTimeout && all_zero(ws));
  // after a clear (status and slots zero) results are exact again
  ws = Workspace(3);
  r = run_call(ws, e, 8, 0.0f);
  CHECK(r[0] == 15.0f && all_zero(ws) && ws.status == 0);
  std::printf("ok protocol\n");
}

int main(int argc, char** argv) {
  const bool quick = argc > 1 && std::strcmp(argv[1], "--quick") == 0;
  chunk_rules();
  protocol();
  if (!quick) encoding_exhaustive();
  return fails ? 1 : 0;
}
