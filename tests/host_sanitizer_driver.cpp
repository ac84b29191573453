// Host-only exercise of the C ABI (include/cdnaqgemv.h) under AddressSanitizer
// and UndefinedBehaviorSanitizer: every argument check, the variant and
// alias lists (with short buffers), the overlap checks of single and grouped
// calls (5000 problems), the quantizer and timing argument checks,
// describe over every operator and size class, and prepared launches
// (cq_prepare over every operator; cq_launch_prepared only on records it
// refuses).  Nothing here launches a
// kernel or touches a GPU: every call fails its host-side checks first or
// only plans.  Built and run by tests/test_host_sanitizers_cpu.py.
#include "cdnaqgemv.h"
#include <cstdio>
#include <cstring>
#include <cstdint>
#include <vector>
int main() {
    char buf[4096];
    for (int op : {CQ_OP_INT4GEMV, CQ_OP_QGEMV, CQ_OP_GEMV_F16, CQ_OP_GEMV_F32, 7})
        for (int which : {CQ_LIST_NORMAL, CQ_LIST_ALL, CQ_LIST_QUARANTINED, CQ_LIST_ALIASES, 9}) {
            int need = cq_variants(op, which, nullptr, 0);
            if (need > 0) { std::vector<char> b(need); cq_variants(op, which, b.data(), b.size()); cq_variants(op, which, b.data(), 3); }
        }
    const void* P = (const void*)0x10000;
    void* Y = (void*)0x90000000;
    // argument errors
    cq_int4gemv(nullptr, P, P, P, Y, 8, 128, nullptr);
    cq_int4gemv("nope", P, P, P, Y, 8, 128, nullptr);
    cq_int4gemv("int4gemv_cdna4", P, P, P, Y, 8, 100, nullptr);
    cq_int4gemv("int4gemv_cdna4", P, P, P, (void*)P, 8, 128, nullptr);   // overlap
    cq_qgemv("qgemv_cdna4", nullptr, P, P, Y, 8, 16, nullptr);
    cq_gemv("gemv_cdna4", 5, P, P, Y, 8, 16, nullptr);
    cq_gemv("gemv_cdna4", CQ_DTYPE_F32, P, P, (void*)P, 8, 16, nullptr);
    std::printf("last: %s\n", cq_last_error());
    // grouped with conflicts, many problems
    std::vector<cq_gemv_problem_t> pr(5000);
    for (size_t i = 0; i < pr.size(); ++i) {
        pr[i].w = (const void*)(0x100000000ull + i * 0x10000); pr[i].scale = (const void*)(0x300000000ull + i * 0x1000);
        pr[i].x = (const void*)0x200000000ull; pr[i].y = (void*)(0x500000000ull + i * 0x1000); pr[i].n = 8;
    }
    pr.back().y = (void*)((const char*)pr[7].w + 4);
    cq_int4gemv_grouped("int4gemv_cdna4", pr.data(), (int64_t)pr.size(), 128, nullptr);
    std::printf("grouped: %s\n", cq_last_error());
    cq_int4gemv_grouped("int4gemv_cdna4", nullptr, 3, 128, nullptr);
    cq_int4gemv_grouped("int4gemv_cdna4", pr.data(), 0, 128, nullptr);
    // quantize argument errors
    cq_int4_quantize(P, (void*)P, Y, 4, 128, CQ_SCALE_RCP, nullptr);
    cq_q8_quantize(P, Y, (void*)0x1002, 4, 16, CQ_SCALE_DIV, nullptr);
    cq_quantize_vectorized(CQ_OP_INT4GEMV, P, Y, 4, 128);
    cq_quantize_vectorized(9, P, Y, 4, 128);
    // timing argument errors
    cq_timing_t t; double tot;
    cq_native_timing(CQ_OP_INT4GEMV, "int4gemv_cdna4", P, P, P, Y, 8, 128, nullptr, -1, 1, 1, nullptr, &t);
    cq_pool_timing(CQ_OP_INT4GEMV, "int4gemv_cdna4", nullptr, nullptr, nullptr, nullptr, 1, 8, 128, nullptr, 0, 0.0, 0.0, 1, nullptr, &tot, nullptr);
    const void* one[1] = {P};
    cq_pool_timing(CQ_OP_INT4GEMV, "int4gemv_cdna4", one, one, one, (void* const*)one, 1, 8, 128, nullptr, 0, -1.0, 0.0, 1, nullptr, &tot, nullptr);
    const void* bufs[2] = {(const void*)0x1000, (const void*)0x2008};
    cq_read_ceiling(bufs, 2, 4096, Y, nullptr, 0, 0.0, 0.0, 1, &tot);
    cq_launch_floor(0, 256, Y, nullptr, 0, 0.0, 0.0, 1, &tot);
    cq_launch_floor(256, 256, Y, nullptr, 0, 0.0, 1e7, 1, &tot);
    // timeline: refused before any launch (null, non-LDS plan, small or
    // overlapping stamp buffer)
    {
        const void* tw[1] = {(const void*)0x10000000};
        const void* ts[1] = {(const void*)0x20000000};
        const void* tx[1] = {(const void*)0x30000000};
        void* ty[1] = {(void*)0x40000000};
        const void* tw_bad[1] = {(const void*)0x10000001};
        int64_t waves = 0; double tpu = 0;
        cq_int4_timeline("int4gemv_cdna4", tw, ts, tx, ty, 1, 4096, 4096, nullptr, 0, 0.0, 0.0, 2,
                         nullptr, 1 << 20, &waves, &tpu, &tot);
        cq_int4_timeline("int4gemv_cdna4", tw_bad, ts, tx, ty, 1, 4096, 4096, nullptr, 0, 0.0, 0.0, 2,
                         (uint64_t*)0x50000000, 1 << 20, &waves, &tpu, &tot);
        cq_int4_timeline("int4gemv_cdna4", tw, ts, tx, ty, 1, 4096, 4096, nullptr, 0, 0.0, 0.0, 2,
                         (uint64_t*)0x50000000, 7, &waves, &tpu, &tot);
        cq_int4_timeline("int4gemv_cdna4", tw, ts, tx, ty, 1, 4096, 4096, nullptr, 0, 0.0, 0.0, 2,
                         (uint64_t*)0x107FFFF8, int64_t(1) << 40, &waves, &tpu, &tot);
        cq_int4_timeline("int4gemv_cdna4", tw, ts, tx, ty, 1, 4096, 4096, nullptr, 0, 0.0, 0.0,
                         INT64_MAX, (uint64_t*)0x50000000, INT64_MAX, &waves, &tpu, &tot);
        std::printf("timeline: %s\n", cq_last_error());
    }
    // describe, every op and size class
    for (int op : {CQ_OP_INT4GEMV, CQ_OP_QGEMV, CQ_OP_GEMV_F16, CQ_OP_GEMV_F32})
        for (int64_t n : {1, 7, 4096, 8192, 1 << 20})
            for (int64_t k : {16, 128, 4096, 11008, 28672, 65536}) {
                const char* v = op == CQ_OP_INT4GEMV ? "int4gemv_cdna4" : op == CQ_OP_QGEMV ? "qgemv_cdna4" : "gemv_lds_tiled";
                int need = cq_describe_launch(op, v, n, k, (const void*)0x1000, (const void*)0x2000, nullptr, 0);
                if (need > 0) { std::vector<char> b(need); cq_describe_launch(op, v, n, k, (const void*)0x1000, (const void*)0x2000, b.data(), b.size()); }
                cq_describe_launch(op, v, n, k, (const void*)0x1000, (const void*)0x2000, buf, 5);
            }
    cq_vec_contract_ok(CQ_OP_INT4GEMV, P, P, 128);
    // prepared launches: checks, plans and records only; the launch entry
    // point is only handed records it must refuse
    cq_prepared_t rec;
    for (int op : {CQ_OP_INT4GEMV, CQ_OP_QGEMV, CQ_OP_GEMV_F16, CQ_OP_GEMV_F32})
        for (int64_t k : {16, 128, 4096, 28672}) {
            const char* v = op == CQ_OP_INT4GEMV ? "int4gemv_cdna4" : op == CQ_OP_QGEMV ? "qgemv_cdna4" : "gemv_cdna4";
            cq_prepare(op, v, (const void*)0x10000000, (const void*)0x20000000, (const void*)0x30000000,
                       (void*)0x40000000, 4096, k, &rec);
        }
    cq_prepare(CQ_OP_INT4GEMV, "nope", P, P, P, Y, 8, 128, &rec);
    cq_prepare(CQ_OP_INT4GEMV, "int4gemv_cdna4", P, P, P, Y, 8, 128, nullptr);
    cq_launch_prepared(nullptr, nullptr);
    cq_launch_prepared(&rec, nullptr);                 // zeroed by the failed prepare
    cq_prepare(CQ_OP_QGEMV, "qgemv_cdna4", (const void*)0x10000000, (const void*)0x20000000,
               (const void*)0x30000000, (void*)0x40000000, 64, 64, &rec);
    rec.opaque[3] ^= 4;                                 // damaged: refused by its seal
    cq_launch_prepared(&rec, nullptr);
    std::printf("prepared: %s\n", cq_last_error());
    std::printf("version %s\ndone\n", cq_version());
    return 0;
}
