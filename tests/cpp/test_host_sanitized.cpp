// Host code of the KV decode path under the address and undefined-behaviour
// sanitizers (built by tests/test_host_sanitizers.py with g++, no GPU):
//  - the decode launch planner (tiny-llm_amd/csrc/attn_plan.cpp) on random
//    and extreme length sets, including the inline-metadata packing;
//  - the CPU oracle (oracle/kv_oracle.c, test infrastructure) through every
//    entry point on small inputs: bookkeeping and append, gather, decode and
//    prefill attention, softmax, attention weights, W8A16, add_inplace.
// Each check prints "ok <name>"; any failure aborts with a message, and any
// sanitizer report aborts the program (-fno-sanitize-recover=all).
#include "attn_plan.h"
#include "kv_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

using namespace tiny_llm::detail;

#define CHECK(c)                                                                                   \
    do {                                                                                           \
        if (!(c)) {                                                                                \
            std::fprintf(stderr, "check failed: %s (%s:%d)\n", #c, __FILE__, __LINE__);          \
            std::abort();                                                                          \
        }                                                                                          \
    } while (0)

static void planner_random() {
    std::mt19937_64 rng(20261201);
    int             fused = 0;
    for (int it = 0; it < 600; ++it) {
        // every fifth plan: near-uniform lengths, up to one 8-head group per CU
        const int n = it % 5 == 4 ? 1 + (int)(rng() % 128) : (int)(rng() % 700);
        std::vector<int32_t> lens((size_t)n);
        const int kind = it % 4;
        for (auto &l : lens) {
            if (it % 5 == 4) l = (int32_t)(7400 + rng() % 800);
            else if (kind == 0) l = (int32_t)(rng() % 65536);
            else if (kind == 1) l = (int32_t)(1 + rng() % 300);
            else if (kind == 2) l = 8193;
            else l = (int32_t)(rng() % 40000);
        }
        int hkv = 1 << (rng() % 6);
        int cus = 1 + (int)(rng() % 300);
        if (it % 5 == 4) { // CUs a multiple of the 8-head groups, or a few more
            hkv = 8 << (rng() % 2);
            const int groups = n * hkv / 8;
            cus = groups * (1 + (int)(rng() % 4)) + (int)(rng() % 3);
        }
        const int forced = (rng() % 3 == 0) ? 256 * (1 + (int)(rng() % 40)) : 0;
        const int fuse = (int)(rng() % 2) ? 1 << (rng() % 4) : 0; // 0, or 1 (auto), 2, 4, 8
        WorkList wl;
        plan_work_list(n ? lens.data() : nullptr, n, hkv, cus, forced, fuse, wl);
        CHECK(wl.chunk % kPlanQuantum == 0 && wl.chunk >= kPlanQuantum);
        CHECK((int)wl.part_base.size() == n + 1);
        CHECK((int)wl.work.size() == 2 * wl.n_work);
        if (wl.fused_chunked) { // head-fused over the chunk plan's items
            if (fuse == 1)
                CHECK(wl.fused_heads == 2 && hkv % 2 == 0 &&
                      plan_waves((int64_t)wl.n_work * hkv, cus, 0) == 4);
            else
                CHECK((fuse == 2 || fuse == 4 || fuse == 8) && wl.fused_heads == fuse && hkv % fuse == 0);
        }
        if (wl.fused_heads && !wl.fused_chunked) { // interleaved items, chunk-major order
            const int hpw = wl.fused_heads;
            CHECK(fuse && !forced && n > 0 && hkv % hpw == 0 && !wl.any_empty);
            CHECK(hpw == 2 || hpw == 4 || hpw == 8);
            const int nch = wl.n_work / n;
            CHECK(nch >= 1 && nch <= kPlanFusedMaxItems && wl.n_work == n * nch);
            CHECK(wl.any_multi == (nch > 1));
            CHECK((int64_t)n * (hkv / hpw) * nch <= cus);
            for (int w = 0; w < wl.n_work; ++w)
                CHECK(wl.work[2 * (size_t)w] == w % n && wl.work[2 * (size_t)w + 1] == w / n);
            for (int i = 0; i <= n; ++i) CHECK(wl.part_base[(size_t)i] == i * nch);
            for (int i = 0; i < n; ++i) CHECK(lens[(size_t)i] >= 1 && lens[(size_t)i] <= wl.chunk);
            ++fused;
            continue;
        }
        std::vector<int> seen((size_t)wl.n_work, 0);
        int prev = INT32_MAX;
        for (int w = 0; w < wl.n_work; ++w) {
            const int i = wl.work[2 * (size_t)w], c = wl.work[2 * (size_t)w + 1];
            CHECK(i >= 0 && i < n);
            CHECK(c >= 0 && wl.part_base[(size_t)i] + c < wl.part_base[(size_t)i + 1]);
            seen[(size_t)(wl.part_base[(size_t)i] + c)]++;
            const int len = std::min(wl.chunk, lens[(size_t)i] - c * wl.chunk);
            CHECK(len > 0 && len <= prev);
            prev = len;
        }
        for (int s : seen) CHECK(s == 1);
        InlineMeta m;
        std::vector<int32_t> rows((size_t)n);
        for (int i = 0; i < n; ++i) rows[(size_t)i] = (int32_t)(rng() % 1300);
        const bool full = n > 0 && inline_words(wl, n, true) <= kInlineWords;
        const int  cw = n ? inline_words_compact(lens.data(), wl, rows.data(), n) : -1;
        const bool fits = pack_inline(n ? lens.data() : nullptr, wl, n ? rows.data() : nullptr, n, m);
        CHECK(fits == (full || (cw > 0 && cw <= kInlineWords)));
        if (fits && !m.compact) {
            CHECK(full && m.off_rows + n <= kInlineWords);
            CHECK(std::equal(lens.begin(), lens.end(), m.w));
            CHECK(std::equal(rows.begin(), rows.end(), m.w + m.off_rows));
        }
        if (fits && m.compact) { // decode as the kernel does
            CHECK(!full && !wl.any_multi && !wl.any_empty && wl.n_work == n);
            for (int k = 0; k < n; ++k) {
                const uint32_t ord = (uint32_t)m.w[m.off_work + (k >> 1)];
                const int      e = (int)((ord >> ((k & 1) * 16)) & 0xffffu);
                CHECK(e == wl.work[2 * (size_t)k] && wl.work[2 * (size_t)k + 1] == 0);
                CHECK((int)((uint32_t)m.w[e] & 0xffffu) == lens[(size_t)e]);
                CHECK((int)((uint32_t)m.w[e] >> 16) == rows[(size_t)e]);
            }
        }
        const int nw = plan_waves((int64_t)wl.n_work * hkv, cus, 0);
        CHECK(nw == 4 || nw == 8);
    }
    CHECK(fused > 10);
    std::printf("ok planner_random (%d head-fused plans)\n", fused);
}

static uint16_t rnd_h(std::mt19937_64 &rng) {
    std::normal_distribution<float> nd(0.f, 1.f);
    return orc_f2h(nd(rng));
}

static void oracle_kv_and_attention() {
    std::mt19937_64 rng(7);
    const int L = 2, H = 2, D = 64, M = 96, S = 5;
    orc_kv_config cfg = {L, H, D, M, S};
    char          err[256];
    orc_kv       *kv = nullptr;
    CHECK(orc_kv_create(&cfg, &kv, err, sizeof err) == 0);
    std::vector<int> ids;
    std::vector<int32_t> lens;
    for (int s = 0; s < S; ++s) {
        int id = -1;
        CHECK(orc_kv_allocate(kv, M, &id, err, sizeof err) == 0);
        const int n = 1 + (int)(rng() % (M - 1));
        std::vector<uint16_t> k((size_t)n * H * D), v(k.size());
        for (auto &x : k) x = rnd_h(rng);
        for (auto &x : v) x = rnd_h(rng);
        for (int l = 0; l < L; ++l) CHECK(orc_kv_append(kv, id, l, k.data(), v.data(), n, err, sizeof err) == 0);
        CHECK(orc_kv_advance(kv, id, n, err, sizeof err) == 0);
        ids.push_back(id);
        lens.push_back(n);
    }
    int extra = -1;
    CHECK(orc_kv_allocate(kv, M, &extra, err, sizeof err) != 0); // exhausted
    CHECK(orc_kv_used(kv) + orc_kv_free(kv) == orc_kv_total(kv));
    // view of layer 1, rows = slots
    std::vector<int32_t> bt((size_t)S);
    for (int s = 0; s < S; ++s) bt[(size_t)s] = orc_kv_slot_of(kv, ids[(size_t)s]);
    const size_t per_layer = (size_t)H * M * D;
    uint16_t    *pool = orc_kv_pool(kv);
    orc_kv_view  view = {pool + 2 * per_layer, pool + 3 * per_layer, bt.data(), 1, 30,
                         (int64_t)(2 * L * per_layer), H * D, D};
    const int    G = 4, Hq = H * G;
    std::vector<uint16_t> q((size_t)S * Hq * D), o16(q.size());
    std::vector<float>    o32(q.size());
    for (auto &x : q) x = rnd_h(rng);
    orc_attn_decode_gqa(q.data(), &view, lens.data(), S, Hq, H, D, 0.125f, o32.data(), o16.data(), 2);
    for (float x : o32) CHECK(std::isfinite(x));
    std::vector<int32_t> one(lens.size(), 1);
    orc_attn_decode_gqa(q.data(), &view, one.data(), S, Hq, H, D, 0.125f, o32.data(), o16.data(), 1);
    // S = 1: o = v_0 / (1 + 1e-6) for every head of the group
    for (int s = 0; s < S; ++s)
        for (int h = 0; h < Hq; ++h)
            for (int d = 0; d < D; ++d) {
                const size_t off = (size_t)bt[(size_t)s] * 2 * L * per_layer + 3 * per_layer + (size_t)(h / G) * D + d;
                const float  v0 = orc_h2f(pool[off]);
                CHECK(std::fabs(o32[((size_t)s * Hq + h) * D + d] - v0 / (1.f + 1e-6f)) <= 1e-6f * std::fabs(v0) + 1e-7f);
            }
    const int smax = M;
    std::vector<uint16_t> g((size_t)S * H * smax * D);
    orc_kv_gather(&view, 0, lens.data(), S, H, D, smax, g.data());
    orc_kv_gather(&view, 1, lens.data(), S, H, D, smax, g.data());
    for (int s = 0; s < S; ++s) CHECK(orc_kv_release(kv, ids[(size_t)s], err, sizeof err) == 0);
    CHECK(orc_kv_release(kv, ids[0], err, sizeof err) != 0);
    CHECK(orc_kv_active(kv) == 0);
    orc_kv_destroy(kv);
    std::printf("ok oracle_kv_and_attention\n");
}

static void oracle_prefill_softmax_weights() {
    std::mt19937_64 rng(11);
    const int B = 2, H = 3, S = 33, D = 32;
    std::vector<uint16_t> q((size_t)B * H * S * D), k(q.size()), v(q.size()), o16(q.size());
    std::vector<float>    o32(q.size());
    for (auto *a : {&q, &k, &v})
        for (auto &x : *a) x = rnd_h(rng);
    orc_attention_prefill(q.data(), k.data(), v.data(), o32.data(), o16.data(), 0.17f, B, H, S, D, 2);
    std::vector<uint16_t> dq((size_t)B * H * D), dk((size_t)B * H * S * D);
    orc_attention_decode(dq.data(), k.data(), v.data(), o32.data(), o16.data(), 0.17f, B, H, S, D);
    std::vector<uint16_t> sm((size_t)7 * S), sm16(sm.size());
    std::vector<float>    sm32(sm.size());
    for (auto &x : sm) x = rnd_h(rng);
    orc_softmax(sm.data(), sm32.data(), sm16.data(), 7, S);
    for (int r = 0; r < 7; ++r) {
        double t = 0;
        for (int j = 0; j < S; ++j) t += sm32[(size_t)r * S + j];
        CHECK(std::fabs(t - 1.0) < 1e-4);
    }
    std::vector<uint16_t> w16((size_t)B * H * S * S);
    std::vector<float>    w32(w16.size());
    orc_get_attention_weights(q.data(), k.data(), w32.data(), w16.data(), 0.17f, B, H, S, S, D, 1);
    for (int i = 0; i < S; ++i)
        for (int j = i + 1; j < S; ++j) CHECK(w32[(size_t)i * S + j] == 0.f);
    std::printf("ok oracle_prefill_softmax_weights\n");
}

static void oracle_w8a16() {
    std::mt19937_64 rng(13);
    const int M = 3, N = 40, K = 70, gs = 32;
    std::vector<uint16_t> x((size_t)M * K), s((size_t)((K + gs - 1) / gs) * N), o16((size_t)M * N),
        hsum(o16.size());
    std::vector<int8_t> w((size_t)K * N);
    std::vector<float>  o32(o16.size());
    for (auto &a : x) a = rnd_h(rng);
    for (auto &a : s) a = orc_f2h(0.01f);
    for (auto &a : w) a = (int8_t)(rng() % 255 - 127);
    orc_w8a16_matmul(x.data(), w.data(), s.data(), o32.data(), o16.data(), M, N, K, gs);
    for (auto &a : hsum) a = rnd_h(rng);
    orc_add_inplace(hsum.data(), o16.data(), hsum.size());
    std::vector<uint16_t> in(1000), back(1000);
    std::vector<float>    f(1000);
    for (size_t i = 0; i < in.size(); ++i) in[i] = (uint16_t)(rng() & 0x7bff);
    orc_h2f_n(in.data(), f.data(), in.size());
    orc_f2h_n(f.data(), back.data(), f.size());
    CHECK(in == back);
    std::vector<uint16_t> nrm(513);
    orc_fill_normal_f16(99, 0.5f, nrm.data(), nrm.size());
    std::printf("ok oracle_w8a16_and_fp16\n");
}

int main() {
    planner_random();
    oracle_kv_and_attention();
    oracle_prefill_softmax_weights();
    oracle_w8a16();
    return 0;
}
