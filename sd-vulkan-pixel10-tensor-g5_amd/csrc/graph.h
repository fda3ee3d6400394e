// Graph execution helpers shared by the UNet, TAESD and CLIP graphs: one Exec walks a
// network's ops either without launching (sizing the activation arena), under stream
// capture (building the HIP graph), or eagerly with every kernel timed on its own.
#pragma once

#include "engine.h"

#include <cstdio>
#include <string>
#include <vector>

namespace sdu {

struct ProfRec {
    std::string cat, kern, shape;
    double flops, bytes;
    hipEvent_t e0, e1;
};

// Times every kernel launch on its own: the launch goes through hipExtLaunchKernelGGL
// with a start and a stop event of its own (SDU_LAUNCH), which record the start and end
// of that kernel's execution.  Each kernel runs once, so the profiled pass computes the
// same values as a forward.
struct EventTimer : KernelTimer {
    hipStream_t s;
    std::string cat, shape;
    std::vector<ProfRec> recs;
    void run(const char* kernel, double flops, double bytes, void (*fn)(const void*), const void* arg) override {
        ProfRec pr;
        pr.cat = cat; pr.kern = kernel; pr.shape = shape;
        pr.flops = flops; pr.bytes = bytes;
        hipEventCreate(&pr.e0);
        hipEventCreate(&pr.e1);
        g_launch_ev0 = pr.e0;
        g_launch_ev1 = pr.e1;
        fn(arg);
        g_launch_ev0 = g_launch_ev1 = nullptr;
        recs.push_back(pr);
    }
};

struct Exec {
    Ctx& c;
    hipStream_t s;
    Arena* ar;
    int B;
    bool dry = false;
    float* gemm_ws = nullptr;
    size_t gemm_ws_need = 0;
    double* gn_acc = nullptr;  // next free GroupNorm accumulator slot (zeroed per forward)
    double* st_next = nullptr;  // per-channel output statistics pool (zeroed per forward)
    double* st_end = nullptr;
    // A forward clears its statistics pool in the launch that stages its inputs, outside
    // the graph (stats_outside): the pool's address and size are recorded here instead of
    // a fill kernel being captured.
    bool stats_outside = false;
    void* stats_pool = nullptr;
    size_t stats_bytes = 0;
    hipError_t err = hipSuccess;
    EventTimer* timer = nullptr;  // eager profiling only

    template <class T>
    T* alloc(size_t n) { return (T*)ar->alloc(n * sizeof(T)); }

    // One op: `cat` names the op category; the kernels it launches report their own
    // names, FLOPs and bytes to the timer when profiling.
    template <class F>
    void run(const char* cat, F&& launch, const std::string& shape = std::string()) {
        if (dry || err != hipSuccess) return;
        if (timer) { timer->cat = cat; timer->shape = shape; }
        hipError_t e = launch();
        if (e != hipSuccess) err = e;
    }
};

inline GemmArgs dense_args(const f16* A, int lda, int M, int N, int K, const f16* W, void* C, int ldc) {
    GemmArgs a{};
    a.M = M; a.N = N; a.K = K;
    a.amode = A_DENSE;
    a.A = A; a.lda = lda; a.K1 = K;
    a.Wt = W;
    a.C = C; a.ldc = ldc;
    a.out_mode = OUT_F16;
    return a;
}

// 3x3 conv (pad 1) as implicit GEMM; returns output spatial size via Ho/Wo.
inline GemmArgs conv3_args(const f16* x, int B, int Hin, int Win, int Cin, int Cout, int stride,
                           int ups, const f16* W, void* y) {
    GemmArgs a{};
    a.amode = A_CONV3;
    a.A = x;
    a.Bn = B; a.Hin = Hin; a.Win = Win; a.Cin = Cin;
    a.stride = stride; a.upsample = ups;
    a.Ho = ups ? 2 * Hin : (stride == 2 ? (Hin - 1) / 2 + 1 : Hin);
    a.Wo = ups ? 2 * Win : (stride == 2 ? (Win - 1) / 2 + 1 : Win);
    a.M = B * a.Ho * a.Wo; a.N = Cout; a.K = 9 * Cin;
    a.Wt = W;
    a.C = y; a.ldc = Cout;
    a.out_mode = OUT_F16;
    return a;
}

inline void gemm(Exec& E, const char* cat, const GemmArgs& a) {
    const size_t ws = gemm_workspace_bytes(a);
    if (ws > E.gemm_ws_need) E.gemm_ws_need = ws;
    char shape[96];
    snprintf(shape, sizeof shape, "%s M=%d N=%d K=%d geglu=%d", a.amode == A_CONV3 ? "conv3" : a.ln_colsum ? "dense_ln" : "dense",
             a.M, a.N, a.K, a.geglu);
    E.run(cat, [&] { return gemm_launch(a, E.gemm_ws, E.s); }, shape);
}

// An activation with, when its producing GEMM kept them, the per-channel sums and sums
// of squares [B][C][2] of its values (for the GroupNorm that reads it).
struct Act {
    const f16* p;
    const double* st;
};

// Statistics slot for a GEMM output of N channels over images of HW pixels, or null
// (then the GroupNorm that reads the output computes its own statistics).
inline void want_stats(Exec& E, GemmArgs& a, int HW) {
    const size_t n = (size_t)E.B * a.N * 2;
    // up to 32x32 pixels the GroupNorm's own single-kernel statistics pass (one block
    // per group and image) costs less than the epilogue statistics and their apply
    if (HW <= 1024 || !gemm_stats_supported(HW) || E.st_next == nullptr || E.st_next + n > E.st_end) return;
    a.stats = E.st_next;
    a.stats_hw = HW;
    E.st_next += n;
}

// GroupNorm (32 groups, epsilon eps) of concat(x, x2) over C1 + C2 channels, optionally
// followed by SiLU: from the producers' epilogue statistics when both kept them, else
// with its own statistics pass (accumulator slot from E.gn_acc).
inline void group_norm_op(Exec& E, Act x, Act x2, int C1, int C2, const f16* g, const f16* b, f16* y, int HW,
                          int silu, float eps) {
    const int G = 32;
    char shape[48];
    snprintf(shape, sizeof shape, "HW=%d C=%d", HW, C1 + C2);
    if (x.st && (C2 == 0 || x2.st)) {
        E.run(silu ? "groupnorm_silu" : "groupnorm", [&] {
            return groupnorm_apply_stats_launch(x.p, x2.p, C1, C2, x.st, x2.st, g, b, y, E.B, HW, G, eps, silu,
                                                E.s);
        }, shape);
        return;
    }
    double* acc = E.gn_acc;
    E.gn_acc += (size_t)E.B * G * 2;
    E.run(silu ? "groupnorm_silu" : "groupnorm", [&] {
        return groupnorm_launch(x.p, x2.p, C1, C2, g, b, y, E.B, HW, G, eps, silu, acc, E.s);
    }, shape);
}

// A planned graph of an auxiliary network for one input shape (`key`): activation arena,
// GEMM workspace, fixed input / output staging buffers and the captured HIP graph.
struct AuxState {
    std::vector<int> key;
    uint64_t last_use = 0;
    char* arena = nullptr;
    size_t arena_bytes = 0;
    float* gemm_ws = nullptr;
    void* in = nullptr;
    void* out = nullptr;
    size_t in_bytes = 0, out_bytes = 0;
    hipGraphExec_t exec = nullptr;
};
typedef void (*AuxBody)(Exec& E, AuxNet& n, AuxState& S);
// The state for `key`, planned on first use (sizing pass, allocation, capture of `body`
// on the context's stream); at most 8 per network, least recently used evicted.
AuxState* aux_state(Ctx& c, AuxNet& n, const std::vector<int>& key, int B, size_t in_bytes, size_t out_bytes,
                    AuxBody body, int* st);

inline int hip_fail(Ctx& c, hipError_t e, const char* what) {
    return set_err(&c, SDU_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace sdu
