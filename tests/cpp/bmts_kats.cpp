// bmts_kats.cpp - the reference's BMTS format tests (bmts.rs:433-509) and
// HadRuntime rules (qwen35.rs:603-613) against the C++ host mirror
// (include/ouro/bmts.hpp).  Host only: nothing here touches a device.
// Usage: bmts_kats <scratch directory>; exit status 0 when all pass.
#include <cstdio>
#include <fstream>
#include <functional>
#include <string>
#include <vector>

#include "../../include/ouro/bmts.hpp"

using namespace ouro;

static int g_failed = 0;
static std::string g_dir;

#define EXPECT(cond)                                                                 \
    do {                                                                             \
        if (!(cond)) {                                                               \
            std::printf("    expectation failed: %s (line %d)\n", #cond, __LINE__); \
            throw std::runtime_error("expectation failed");                         \
        }                                                                            \
    } while (0)

template <typename F>
static bool throws(F &&f) {
    try {
        f();
    } catch (const Error &) {
        return true;
    }
    return false;
}

static void run(const char *name, const std::function<void()> &fn) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const std::exception &e) {
        ++g_failed;
        std::printf("FAIL %s: %s\n", name, e.what());
    }
}

static void write_raw(const std::string &path, const std::string &bytes) {
    std::ofstream(path, std::ios::binary).write(bytes.data(), static_cast<std::streamsize>(bytes.size()));
}

static std::string header(uint16_t version, uint32_t n, uint32_t meta_len) {
    std::string h(16, '\0');
    const uint32_t magic = bmts::kMagic;
    const uint16_t node = 1;
    std::memcpy(&h[0], &magic, 4);
    std::memcpy(&h[4], &version, 2);
    std::memcpy(&h[6], &node, 2);
    std::memcpy(&h[8], &n, 4);
    std::memcpy(&h[12], &meta_len, 4);
    return h;
}

static void test_bmts_roundtrip() {  // bmts.rs:433-496
    const std::string path = g_dir + "/shard_1.bmts";
    std::vector<uint8_t> blob(64);
    for (int i = 0; i < 64; ++i) blob[i] = static_cast<uint8_t>(i);
    bmts::Tensor q{"blk.0.attn_q.weight", {8, 8}, 34, 0, 32}, k{"blk.0.attn_k.weight", {8, 8}, 34, 32, 32};
    bmts::write_shard(path, 1, {q, k}, blob);
    bmts::Shard shard(path);
    EXPECT(shard.node() == 1);
    EXPECT(shard.tensors().size() == 2);
    EXPECT(shard.data_len() == 64);
    EXPECT(shard.read_tensor("blk.0.attn_q.weight") == std::vector<uint8_t>(blob.begin(), blob.begin() + 32));
    EXPECT(shard.read_tensor("blk.0.attn_k.weight") == std::vector<uint8_t>(blob.begin() + 32, blob.end()));
    EXPECT(throws([&] { shard.read_tensor("missing"); }));
    const auto sub = shard.read_span("blk.0.attn_q.weight", 8, 16);
    EXPECT(sub.second == 16 && std::memcmp(sub.first, blob.data() + 8, 16) == 0);
    const auto full = shard.read_span("blk.0.attn_q.weight", 0, 32);
    EXPECT(full.second == 32 && std::memcmp(full.first, blob.data(), 32) == 0);
    EXPECT(throws([&] { shard.read_span("blk.0.attn_q.weight", 0, 33); }));
    size_t out_len = 0, in_len = 0;
    shard.weight_shape("blk.0.attn_q.weight", &out_len, &in_len);
    EXPECT(out_len == 8 && in_len == 8);
}

static void test_bmts_bad_magic() {  // bmts.rs:498-507
    const std::string path = g_dir + "/bad.bmts";
    write_raw(path, std::string(32, '\0'));
    EXPECT(throws([&] { bmts::Shard s(path); }));
}

static void test_bmts_malformed() {
    const std::string meta = "[{\"name\":\"a\",\"shape\":[4],\"dtype\":0,\"offset\":0,\"length\":16}]";
    const std::vector<std::pair<std::string, std::string>> cases = {
        {"short", "OURO"},
        {"truncated_meta", header(1, 1, static_cast<uint32_t>(meta.size() + 10)) + meta},
        {"count_mismatch", header(1, 2, static_cast<uint32_t>(meta.size())) + meta + std::string(16, '\0')},
        {"v2", header(2, 1, 8) + std::string(8, '\0')},
        {"unknown_version", header(7, 1, static_cast<uint32_t>(meta.size())) + meta},
        {"bad_table", header(1, 1, 5) + "[{]]]"},
        {"missing_field", header(1, 1, 14) + "[{\"name\":\"a\"}]"},
    };
    for (const auto &c : cases) {
        const std::string path = g_dir + "/" + c.first + ".bmts";
        write_raw(path, c.second);
        if (!throws([&] { bmts::Shard s(path); })) {
            std::printf("    accepted malformed shard: %s\n", c.first.c_str());
            EXPECT(false);
        }
    }
    // a well-formed table whose tensor runs past the file is refused on access
    const std::string path = g_dir + "/short_data.bmts";
    write_raw(path, header(1, 1, static_cast<uint32_t>(meta.size())) + meta + std::string(8, '\0'));
    bmts::Shard s(path);
    EXPECT(throws([&] { s.tensor_bytes("a"); }));
    // an offset near 2^64 must not wrap back into the header or the table
    const std::string wrap =
        "[{\"name\":\"w\",\"shape\":[4],\"dtype\":0,\"offset\":18446744073709551595,\"length\":16}]";
    const std::string wpath = g_dir + "/wrapped.bmts";
    write_raw(wpath, header(1, 1, static_cast<uint32_t>(wrap.size())) + wrap + std::string(16, '\0'));
    bmts::Shard sw(wpath);
    EXPECT(throws([&] { sw.tensor_bytes("w"); }));
    EXPECT(throws([&] { sw.read_span("w", 0, 16); }));
    // spans near 2^64 inside a valid tensor are refused too
    const std::string okp = g_dir + "/ok.bmts";
    write_raw(okp, header(1, 1, static_cast<uint32_t>(meta.size())) + meta + std::string(16, '\0'));
    bmts::Shard so(okp);
    EXPECT(throws([&] { so.read_span("a", 18446744073709551615ull, 2); }));
    EXPECT(throws([&] { so.read_span("a", 8, 18446744073709551615ull); }));
    // a number past 2^64 - 1 is a parse error of the table (ouro::Error), not std::out_of_range
    const std::string big =
        "[{\"name\":\"b\",\"shape\":[4],\"dtype\":0,\"offset\":99999999999999999999999,\"length\":16}]";
    const std::string bpath = g_dir + "/bignum.bmts";
    write_raw(bpath, header(1, 1, static_cast<uint32_t>(big.size())) + big);
    bool parse_error = false;
    try {
        bmts::Shard sb(bpath);
    } catch (const ouro::Error &) {
        parse_error = true;
    } catch (const std::exception &) {
    }
    EXPECT(parse_error);
}

static void test_had_runtime_offsets() {  // qwen35.rs:603-613
    std::vector<float> signs(2560 + 6912 + 4096, 1.0f);
    HadRuntime had(256, {2560, 6912, 4096}, signs, true);
    EXPECT(had.offset_for(2560) == 0);
    EXPECT(had.offset_for(6912) == 2560);
    EXPECT(had.offset_for(4096) == 2560 + 6912);
    EXPECT(had.gdn_v_grouped() && had.block() == 256);
    EXPECT(throws([&] { had.offset_for(1024); }));
    EXPECT(throws([&] { HadRuntime bad(256, {8, 8}, std::vector<float>(15, 1.0f)); }));
}

int main(int argc, char **argv) {
    g_dir = argc > 1 ? argv[1] : "/tmp";
    run("bmts::test_bmts_roundtrip", test_bmts_roundtrip);
    run("bmts::test_bmts_bad_magic", test_bmts_bad_magic);
    run("bmts::malformed_headers", test_bmts_malformed);
    run("qwen35::had_runtime_offsets", test_had_runtime_offsets);
    std::printf("%d failed\n", g_failed);
    return g_failed ? 1 : 0;
}
