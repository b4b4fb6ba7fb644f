// The batch cache header of the C++ host interface (zkie::write_header /
// read_header, include/zkie_hip.hpp) on the CPU: no device code runs, so
// this program is built with g++ alone and needs no library.
//
// The fixture is the metadata of the reference's own cache round trip
// (crates/zkie-core/src/pcs/whir.rs:875-886: "test-model", "group-0", three
// "layer-i-weight" tables of arity 5, security 32, pow bits 10, digest
// [7; 32]) with a one-digest cap [1, ..., 8], laid out by hand in bincode
// 1.3.3's encoding of the (magic, metadata, commitment) tuple: magic bytes,
// u32 schema version, each string as u64 length + bytes, the identifier
// list as u64 count + strings, four u32, 32 digest bytes, the cap as u64
// count + 8 u64 per digest, all little-endian.
#include <cstdio>
#include <cstdlib>
#include <sstream>
#include <string>

#include "zkie_hip.hpp"

static int g_checks = 0;
#define EXPECT(cond, what)                                      \
    do {                                                        \
        if (!(cond)) {                                          \
            std::printf("FAIL %s (line %d)\n", what, __LINE__); \
            std::exit(1);                                       \
        }                                                       \
        std::printf("ok   %s\n", what);                         \
        g_checks++;                                             \
    } while (0)

static const char* kExpectedHex =
    "5a4b494542434832"                  // "ZKIEBCH2"
    "02000000"                          // schema_version 2
    "0a00000000000000"                  // model_id: 10 bytes
    "746573742d6d6f64656c"              //   "test-model"
    "0700000000000000"                  // group_id: 7 bytes
    "67726f75702d30"                    //   "group-0"
    "0300000000000000"                  // table_ids: 3 strings
    "0e00000000000000" "6c617965722d302d776569676874"  // "layer-0-weight"
    "0e00000000000000" "6c617965722d312d776569676874"  // "layer-1-weight"
    "0e00000000000000" "6c617965722d322d776569676874"  // "layer-2-weight"
    "05000000"                          // table_arity 5
    "03000000"                          // num_tables 3
    "20000000"                          // security_level 32
    "0a000000"                          // pow_bits 10
    "0707070707070707070707070707070707070707070707070707070707070707"  // source_digest
    "0100000000000000"                  // cap: 1 digest
    "0100000000000000" "0200000000000000" "0300000000000000" "0400000000000000"
    "0500000000000000" "0600000000000000" "0700000000000000" "0800000000000000";

static std::string hex(const std::string& s)
{
    static const char* d = "0123456789abcdef";
    std::string h;
    for (unsigned char c : s) {
        h.push_back(d[c >> 4]);
        h.push_back(d[c & 15]);
    }
    return h;
}

int main()
{
    zkie::BatchCacheMetadata m;
    m.model_id = "test-model";
    m.group_id = "group-0";
    m.table_ids = {"layer-0-weight", "layer-1-weight", "layer-2-weight"};
    m.table_arity = 5;
    m.num_tables = 3;
    m.security_level = 32;
    m.pow_bits = 10;
    m.source_digest.fill(7);
    zkie::MerkleCap cap{zkie::Digest{1, 2, 3, 4, 5, 6, 7, 8}};

    std::ostringstream os;
    zkie::write_header(os, m, cap);
    EXPECT(hex(os.str()) == kExpectedHex, "write_header lays the tuple out as bincode 1.3.3 does");

    std::istringstream is(os.str() + "rest");
    const auto back = zkie::read_header(is);
    EXPECT(back.first == m && back.second == cap, "read_header returns the metadata and the cap");
    std::string rest;
    is >> rest;
    EXPECT(rest == "rest", "read_header stops at the end of the header (the prover data follows)");

    auto refused = [](const std::string& bytes) {
        std::istringstream s(bytes);
        try {
            (void)zkie::read_header(s);
        } catch (const zkie::Error&) {
            return true;
        }
        return false;
    };
    std::string bad = os.str();
    bad[7] = '1';  // "ZKIEBCH1"
    EXPECT(refused(bad), "read_header refuses another magic");
    bad = os.str();
    bad[8] = 3;  // schema version 3
    EXPECT(refused(bad), "read_header refuses another schema version");
    EXPECT(refused(os.str().substr(0, 100)), "read_header refuses a short stream");
    bad = os.str();
    bad[12 + 7] = 0x40;  // model_id length 2^62
    EXPECT(refused(bad), "read_header refuses an absurd length instead of allocating it");

    zkie::BatchCacheMetadata wrong = m;
    wrong.num_tables = 2;
    bool threw = false;
    try {
        std::ostringstream o2;
        zkie::write_header(o2, wrong, cap);
    } catch (const zkie::Error&) {
        threw = true;
    }
    EXPECT(threw, "write_header refuses a table count that does not match the identifiers");
    std::printf("ALL PASS %d\n", g_checks);
    return 0;
}
