// UTF-8 piece streaming for the token loop's text output: the app's emit
// (src/xiaoju-pipe/ios/App/XJGlue.c:285-305) hands the UI whole characters
// only. The held-back bytes, the 256-byte cut of a piece and the look-back
// over at most 4 bytes are the app's rules, so callers see the same
// chunks; the code is this library's.
#include "xj_hip.h"

#include <cstring>

namespace {

// Length of the UTF-8 sequence a lead byte starts (1 for ASCII and for bytes
// that cannot lead, as the app treats them).
int seq_len(unsigned char c) { return c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : c >= 0xC0 ? 2 : 1; }

// Bytes of buf[0, n) that end on a character boundary: the last lead byte
// within the final 4 bytes decides whether its character is complete; a run of
// 4 continuation bytes (no lead byte in reach) counts as complete.
int complete_prefix(const char *buf, int n) {
    for (int back = 1; back <= 4 && back <= n; back++) {
        const unsigned char c = (unsigned char)buf[n - back];
        if ((c & 0xC0) == 0x80) continue;   // a continuation byte: look further back
        return seq_len(c) > back ? n - back : n;
    }
    return n;
}

}  // namespace

extern "C" void xjh_utf8_reset(xjh_utf8_state *st) {
    if (st) st->npending = 0;
}

extern "C" int xjh_utf8_emit(xjh_utf8_state *st, const char *piece, int n, xjh_piece_fn cb, void *ctx) {
    char buf[sizeof st->pending + 256];
    const int held = st->npending > 0 && st->npending <= (int)sizeof st->pending ? st->npending : 0;
    if (n < 0) n = 0;
    if (n > 256) n = 256;
    std::memcpy(buf, st->pending, held);
    if (n) std::memcpy(buf + held, piece, n);
    const int total = held + n, ready = complete_prefix(buf, total);
    st->npending = total - ready;   // at most 3 bytes: an incomplete character
    std::memcpy(st->pending, buf + ready, st->npending);
    return ready && cb ? cb(ctx, buf, ready) : 0;
}
