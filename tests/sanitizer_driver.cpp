// Host code under AddressSanitizer and UndefinedBehaviorSanitizer: drives the
// plan authority (csrc/plan.cpp: admission arithmetic, partition rules,
// workspace layouts, rotary tables) and the CPU oracle (oracle/*.c) over
// sweeps of valid and invalid inputs, edge sizes included.  Built and run by
// tests/test_host_sanitizers.py with -fsanitize=address,undefined and
// -fno-sanitize-recover=all, so any out-of-bounds access, overflow of a signed
// type, misaligned access or leak ends the run with a report and a non-zero
// status.  Host only: nothing here touches a GPU.

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "pvlc_internal.hpp"

extern "C" {
#include "pvlc_oracle.h"
}

using namespace pvlc;

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint32_t next_u32() {
    g_state ^= g_state << 13;
    g_state ^= g_state >> 7;
    g_state ^= g_state << 17;
    return static_cast<uint32_t>(g_state >> 16);
}
float next_f32() { return static_cast<float>(next_u32() % 20001) / 10000.0f - 1.0f; }
std::vector<float> randv(size_t n) {
    std::vector<float> v(n);
    for (float &x : v) x = next_f32();
    return v;
}

int g_checks = 0;
void expect(bool ok, const char *what) {
    ++g_checks;
    if (!ok) {
        std::fprintf(stderr, "check failed: %s\n", what);
        std::exit(3);
    }
}

void plans() {
    // Session descriptors: the pinned geometry, wrong dimensions, capacities
    // around the split-span bound, buffer lengths off by one, poison tails.
    const uint32_t dims[][3] = {{16, 2, 128}, {0, 2, 128}, {16, 0, 128}, {16, 2, 0}, {16, 3, 128}, {8, 2, 128},
                                {16, 2, 129}, {0xFFFFFFFFu, 2, 128}};
    const uint32_t caps[] = {1, 2, 7, 16, 1025, 2304, 131040, 131041, 0xFFFFFFFFu};
    for (const auto &d : dims)
        for (uint32_t cap : caps)
            for (uint32_t prefix : {0u, 1u, cap / 2, cap > 0 ? cap - 1 : 0u, cap}) {
                const size_t width = static_cast<size_t>(d[1]) * d[2];
                const size_t n = cap <= 4096 ? static_cast<size_t>(cap) * width : 16;
                std::vector<float> k(n + 1, 0.5f), v(n + 1, 0.25f);
                for (int off : {0, -1, 1}) {
                    pvlc_hip_kv_session_descriptor desc{d[0], d[1], d[2], prefix, cap, k.data(),
                                                        static_cast<size_t>(static_cast<long>(n) + (off < 0 && n == 0 ? 0 : off)),
                                                        v.data(), n};
                    pvlc_hip_kv_session_plan plan{};
                    const pvlc_hip_status st = pvlc_hip_kv_session_plan_create(&desc, &plan);
                    if (st != 0) continue;
                    std::vector<float> q(plan.query_elements + 1), row(plan.key_value_width + 1);
                    for (uint32_t t : {prefix, prefix + 1, cap, cap > 0 ? cap - 1 : 0u}) {
                        for (int qoff : {0, -1}) {
                            pvlc_hip_kv_step_operands ops{q.data(), static_cast<size_t>(plan.query_elements + qoff),
                                                          row.data(), plan.key_value_width, row.data(),
                                                          plan.key_value_width};
                            pvlc_hip_kv_step_plan sp{};
                            (void)pvlc_hip_kv_session_plan_step(&plan, t, &ops, &sp);
                            (void)pvlc_hip_kv_session_plan_step(&plan, t, nullptr, &sp);
                        }
                    }
                }
            }
    for (uint32_t t = 0; t < 140000; t += 97) {
        pvlc_hip_gqa_split_plan sp{};
        (void)pvlc_hip_gqa_split_plan_create(t, 16, 2, 128, &sp);
        (void)pvlc_hip_gqa_split_plan_create(t, 16, 3, 128, &sp);
        (void)pvlc_hip_prefill_plan_check(t, t + 1);
        (void)pvlc_hip_prefill_plan_check(t + 1, t);
    }
    for (uint32_t rows : {0u, 1u, 7u, 256u, 1024u, 103424u, 524280u, 524281u, 0xFFFFFFFFu})
        for (uint32_t cols : {0u, 1u, 1024u, 2048u, 3072u, 4096u}) {
            pvlc_hip_gemv_tiled_plan gp{};
            (void)pvlc_hip_gemv_tiled_plan_create(rows, cols, &gp);
            pvlc_hip_projection_plan pp{};
            for (uint32_t storage : {0u, 1u, 2u})
                if (pvlc_hip_projection_plan_create(rows, cols, 1024, storage, &pp) == 0) {
                    (void)pvlc_hip_projection_validate_capabilities(&pp, storage == 1 ? 1 : 0, 65535);
                    (void)pvlc_hip_projection_validate_capabilities(&pp, 0, 1);
                }
        }
    // Projection operand checks over real buffers, finite and not.
    {
        pvlc_hip_projection_plan pp{};
        expect(pvlc_hip_projection_plan_create(5, 32, 8, 1, &pp) == 0, "projection plan 5x32x8");
        std::vector<float> in(5 * 32, 1.0f), bias(8, 0.0f);
        std::vector<uint16_t> w(32 * 8, 0x3c00);
        expect(pvlc_hip_projection_validate_operands(&pp, in.data(), in.size() * 4, w.data(), w.size() * 2,
                                                     bias.data(), bias.size() * 4) == 0,
               "projection operands");
        in[17] = NAN;
        expect(pvlc_hip_projection_validate_operands(&pp, in.data(), in.size() * 4, w.data(), w.size() * 2,
                                                     bias.data(), bias.size() * 4) != 0,
               "non-finite projection input rejected");
        (void)pvlc_hip_projection_validate_operands(&pp, in.data(), in.size() * 4 - 4, w.data(), w.size() * 2,
                                                    bias.data(), bias.size() * 4);
    }
    // Decode partition rules and workspace layouts over the admissible range.
    for (uint32_t seqs : {1u, 2u, 3u, 18u, 64u, 256u, 2048u, 2049u, 65535u})
        for (uint32_t ctx : {1u, 2u, 16u, 17u, 1025u, 2048u, 2304u, 6144u, 6145u, 8192u, 32768u, 131040u}) {
            const uint32_t p = auto_partition(seqs, ctx);
            expect(p >= 16 && p % 16 == 0 && p <= 4096, "automatic partition in 16..4096");
            const uint32_t parts = auto_workspace_parts(seqs, ctx);
            const DecodeWorkspace w = decode_workspace_layout(seqs, parts);
            expect(w.total >= w.part_o_offset && w.part_stride % 2 == 1, "decode workspace layout");
            (void)single_shot_partition(seqs, ctx);
            (void)decode_shape(p, false);
            (void)decode_shape(p, true);
        }
    for (uint32_t tokens = 0; tokens < 9000; tokens += 37) {
        const PrefillWorkspace w = prefill_workspace_layout(tokens);
        expect(w.total >= w.partial_offset, "prefill workspace layout");
        const uint32_t qblocks = (tokens + 15) / 16;
        for (uint32_t wg = 0; qblocks && wg < prefill_pair_workgroups(qblocks); ++wg) {
            uint32_t g = 0, pair = 0;
            PrefillSegment a{}, b{};
            (void)prefill_pair_segments(wg, qblocks, &g, &pair, &a, &b);
        }
    }
    // Rotary tables (NeoX, then the M-RoPE section selection of raw tables).
    for (uint32_t rows : {1u, 2u, 17u, 300u}) {
        std::vector<float> c(static_cast<size_t>(rows) * 64), s(c.size());
        (void)pvlc_hip_rope_table_f32(500000.0f, 128, rows, c.data(), s.data());
        (void)pvlc_hip_rope_table_f32(-1.0f, 128, rows, c.data(), s.data());
        std::vector<float> raw_c(3 * static_cast<size_t>(rows) * 128), raw_s(raw_c.size());
        for (size_t i = 0; i < raw_c.size(); ++i) raw_c[i] = raw_s[i] = static_cast<float>(i % 64) * 0.01f;
        (void)pvlc_hip_mrope_table_f32(raw_c.data(), raw_s.data(), rows, 16, 24, 24, c.data(), s.data());
        (void)pvlc_hip_mrope_table_f32(raw_c.data(), raw_s.data(), rows, 16, 24, 25, c.data(), s.data());
    }
    // fp16 conversions over every half and a sweep of floats.
    std::vector<uint16_t> halves(65536);
    for (uint32_t i = 0; i < 65536; ++i) halves[i] = static_cast<uint16_t>(i);
    std::vector<float> widened(65536);
    pvlc_hip_f16_to_f32_host(halves.data(), widened.data(), halves.size());
    std::vector<uint16_t> back(65536);
    pvlc_hip_f32_to_f16_host(widened.data(), back.data(), back.size());
    for (uint32_t i = 0; i < 65536; ++i)
        if (!std::isnan(widened[i])) expect(back[i] == halves[i], "fp16 round trip");
}

void oracle() {
    // Decode and causal GQA over small and boundary shapes, including group 1
    // and a single kv head, plus the error paths of short buffers.
    const size_t shapes[][3] = {{16, 2, 128}, {4, 2, 6}, {2, 2, 4}, {3, 1, 5}, {4, 4, 3}};
    for (const auto &sh : shapes)
        for (size_t t : {1u, 2u, 15u, 16u, 17u, 33u, 65u}) {
            const size_t qh = sh[0], kvh = sh[1], d = sh[2];
            std::vector<float> q = randv(qh * d), k = randv(t * kvh * d), v = randv(t * kvh * d), out(qh * d);
            expect(oracle_decode_gqa_f32(q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), t, qh, kvh, d,
                                         out.data()) == 0,
                   "oracle decode");
            (void)oracle_decode_gqa_f32(q.data(), q.size(), k.data(), k.size() - 1, v.data(), v.size(), t, qh, kvh, d,
                                        out.data());
            std::vector<float> cq = randv(t * qh * d), cout(t * qh * d);
            expect(oracle_causal_gqa_f32(cq.data(), cq.size(), k.data(), k.size(), v.data(), v.size(), t, qh, kvh, d,
                                         cout.data()) == 0,
                   "oracle causal");
            std::vector<float> rk = randv(kvh * d), rv = randv(kvh * d);
            std::vector<float> ok((t + 1) * kvh * d), ov((t + 1) * kvh * d);
            expect(oracle_append_kv_f32(k.data(), v.data(), t, rk.data(), rk.size(), rv.data(), rv.size(), kvh, d,
                                        ok.data(), ov.data()) == 0,
                   "oracle append");
            (void)oracle_append_kv_f32(k.data(), v.data(), t, rk.data(), rk.size() - 1, rv.data(), rv.size(), kvh, d,
                                       ok.data(), ov.data());
            std::vector<float> pk(t * kvh * d), pv(t * kvh * d);
            (void)oracle_write_prefill_kv_f32(k.data(), k.size(), v.data(), v.size(), t, kvh, d, pk.data(), pv.data());
            std::vector<float> ind(qh * d);
            oracle_independent_decode_gqa_f32(q.data(), k.data(), v.data(), t, qh, kvh, d,
                                              1.0f / std::sqrt(static_cast<float>(d)), 0, ind.data());
        }
    for (size_t rows : {1u, 3u, 16u})
        for (size_t width : {2u, 6u, 128u}) {
            std::vector<float> x = randv(rows * width);
            std::vector<uint32_t> pos(rows);
            for (size_t r = 0; r < rows; ++r) pos[r] = static_cast<uint32_t>(r * 7);
            (void)oracle_rope_neox_f32(x.data(), x.size(), rows, width, width, pos.data(), pos.size(), 500000.0f);
            (void)oracle_rope_neox_f32(x.data(), x.size(), rows, width, width + 2, pos.data(), pos.size(), 500000.0f);
            (void)oracle_rope_neox_f32(x.data(), x.size(), rows, width, width, pos.data(), pos.size() - 1, 500000.0f);
        }
    {
        std::vector<float> in = randv(5 * 32), w = randv(32 * 8), b = randv(8), out(5 * 8);
        expect(oracle_linear_f32(in.data(), in.size(), 5, 32, w.data(), w.size(), b.data(), b.size(), 8,
                                 out.data()) == 0,
               "oracle linear");
        (void)oracle_linear_f32(in.data(), in.size(), 5, 32, w.data(), w.size() - 1, b.data(), b.size(), 8,
                                out.data());
        std::vector<float> logits = randv(1000);
        logits[17] = NAN;
        logits[99] = INFINITY;
        uint32_t idx = 0, bits = 0;
        (void)oracle_top1_f32(logits.data(), logits.size(), &idx, &bits);
        (void)oracle_top1_f32(logits.data(), 0, &idx, &bits);
    }
    {
        // M-RoPE over an image grid's distinct (t, h, w) tables, sections [16, 24, 24] and a bad split.
        const size_t tokens = 20, qh = 16, kvh = 2, d = 128;
        std::vector<float> q = randv(tokens * qh * d), k = randv(tokens * kvh * d);
        std::vector<float> rc = randv(3 * tokens * d), rs = randv(3 * tokens * d);
        std::vector<float> oq(q.size()), okk(k.size());
        const size_t good[3] = {16, 24, 24}, bad[3] = {16, 24, 25};
        (void)oracle_mrope_f32(q.data(), q.size(), k.data(), k.size(), tokens, qh, kvh, d, rc.data(), rs.data(),
                               rc.size(), good, oq.data(), okk.data());
        (void)oracle_mrope_f32(q.data(), q.size(), k.data(), k.size(), tokens, qh, kvh, d, rc.data(), rs.data(),
                               rc.size(), bad, oq.data(), okk.data());
    }
    for (size_t n : {0u, 1u, 63u, 64u, 65u, 1023u, 1024u, 1025u, 2048u, 5000u}) {
        std::vector<uint8_t> bytes(n + 1);
        for (size_t i = 0; i < n; ++i) bytes[i] = static_cast<uint8_t>(i % 251);
        uint8_t digest[32];
        oracle_blake3(bytes.data(), n, digest);
    }
    std::vector<uint16_t> h(4096);
    oracle_normal_f16(7, 0.5f, h.data(), h.size());
    std::vector<float> f(4096);
    oracle_normal_f32(7, f.data(), f.size());
}

}  // namespace

int main() {
    plans();
    oracle();
    std::printf("sanitizer driver: %d checks passed\n", g_checks);
    return 0;
}
