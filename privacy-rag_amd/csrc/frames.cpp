// The 96-byte public frame header that precedes every payload the reference's
// Channel sends (Channel::send_data / recv_data, native/src/channel.cpp:122-150):
//   [0, 8)    "PRGCF001"
//   [8, 24)   session id, [24, 56) configuration digest
//   [56, 96)  five big-endian u64: sequence, payload bytes, stage, operation,
//             protocol version 1.
// A ciphertext frame's payload is the [component][prime][N] little-endian u64
// layout every praghip entry point takes, so a transport frames device results
// as they are.  Host-only byte work.
#include <cstring>

#include "praghip.h"
#include "host.hpp"

using namespace praghip::host;

namespace {
constexpr unsigned char kMagic[8] = {'P', 'R', 'G', 'C', 'F', '0', '0', '1'};
constexpr uint64_t kVersion = 1;

void put_be64(uint8_t* p, uint64_t x) {
  for (int i = 0; i < 8; ++i) p[i] = uint8_t(x >> (56 - 8 * i));
}
uint64_t get_be64(const uint8_t* p) {
  uint64_t x = 0;
  for (int i = 0; i < 8; ++i) x = (x << 8) | p[i];
  return x;
}
}  // namespace

extern "C" {

int praghip_frame_encode(const praghip_frame_header* h, uint8_t* out) {
  if (!h || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  std::memcpy(out, kMagic, 8);
  std::memcpy(out + 8, h->session, 16);
  std::memcpy(out + 24, h->config, 32);
  put_be64(out + 56, h->sequence);
  put_be64(out + 64, h->size);
  put_be64(out + 72, h->stage);
  put_be64(out + 80, h->operation);
  put_be64(out + 88, kVersion);
  return PRAGHIP_OK;
}

int praghip_frame_decode(const uint8_t* in, praghip_frame_header* h) {
  if (!in || !h) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (std::memcmp(in, kMagic, 8) != 0 || get_be64(in + 88) != kVersion)
    return fail(PRAGHIP_E_SHAPE, "E_FRAME_BINDING");
  std::memcpy(h->session, in + 8, 16);
  std::memcpy(h->config, in + 24, 32);
  h->sequence = get_be64(in + 56);
  h->size = get_be64(in + 64);
  h->stage = get_be64(in + 72);
  h->operation = get_be64(in + 80);
  return PRAGHIP_OK;
}

int praghip_frame_check(const uint8_t* in, const praghip_frame_header* expect) {
  if (!in || !expect) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  praghip_frame_header got;
  if (int rc = praghip_frame_decode(in, &got)) return rc;
  if (std::memcmp(got.session, expect->session, 16) != 0 || std::memcmp(got.config, expect->config, 32) != 0 ||
      got.sequence != expect->sequence || got.size != expect->size || got.stage != expect->stage ||
      got.operation != expect->operation)
    return fail(PRAGHIP_E_SHAPE, "E_FRAME_BINDING");
  return PRAGHIP_OK;
}

}  // extern "C"
