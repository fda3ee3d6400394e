// Planned graphs and weight pools of the auxiliary networks (TAESD decoder, CLIP text
// encoder): the same plan-once / replay scheme as the UNet forward (one sizing pass,
// one allocation, one captured HIP graph per input shape).
#include "graph.h"

#include <algorithm>

namespace sdu {

static void free_aux_state(AuxState* S) {
    if (!S) return;
    if (S->exec) hipGraphExecDestroy(S->exec);
    hipFree(S->arena);
    hipFree(S->gemm_ws);
    hipFree(S->in);
    hipFree(S->out);
    delete S;
}

void aux_free(AuxNet* n) {
    if (!n) return;
    for (AuxState* s : n->states) free_aux_state(s);
    n->states.clear();
    hipFree(n->pool);
    delete n;
}

static int plan_aux(Ctx& c, AuxNet& n, AuxState& S, int B, AuxBody body) {
    Arena ar;
    ar.sizing = true;
    Exec dry{c, c.stream, &ar, B};
    dry.dry = true;
    body(dry, n, S);
    S.arena_bytes = ar.high;
    auto mal = [&](void** p, size_t bytes) { return hipMalloc(p, bytes < 256 ? 256 : bytes); };
    if (mal((void**)&S.arena, S.arena_bytes) != hipSuccess || mal((void**)&S.gemm_ws, dry.gemm_ws_need) != hipSuccess ||
        mal(&S.in, S.in_bytes) != hipSuccess || mal(&S.out, S.out_bytes) != hipSuccess)
        return set_err(&c, SDU_ERR_OOM, "graph state allocation failed");
    hipError_t e;
    if (dry.gemm_ws_need && (e = zero_launch(S.gemm_ws, gemm_counter_bytes(), c.stream)) != hipSuccess)
        return hip_fail(c, e, "gemm workspace");
    ar.sizing = false;
    ar.base = S.arena;
    ar.cap = S.arena_bytes;
    ar.top = ar.high = 0;
    Exec E{c, c.stream, &ar, B};
    E.gemm_ws = S.gemm_ws;
    hipGraph_t g = nullptr;
    if ((e = hipStreamBeginCapture(c.stream, hipStreamCaptureModeThreadLocal)) != hipSuccess)
        return hip_fail(c, e, "begin capture");
    body(E, n, S);
    hipError_t ec = hipStreamEndCapture(c.stream, &g);
    if (E.err != hipSuccess) { if (g) hipGraphDestroy(g); return hip_fail(c, E.err, "kernel launch during capture"); }
    if (ec != hipSuccess) return hip_fail(c, ec, "end capture");
    e = hipGraphInstantiate(&S.exec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(c, e, "graph instantiate");
    return SDU_OK;
}

AuxState* aux_state(Ctx& c, AuxNet& n, const std::vector<int>& key, int B, size_t in_bytes, size_t out_bytes,
                    AuxBody body, int* st) {
    for (AuxState* s : n.states)
        if (s->key == key) {
            s->last_use = ++n.use_clock;
            return s;
        }
    if (n.states.size() >= 8) {
        hipError_t e = hipStreamSynchronize(c.stream);  // the evicted graph may still run
        if (e != hipSuccess) { *st = hip_fail(c, e, "evict state"); return nullptr; }
        auto lru = std::min_element(n.states.begin(), n.states.end(),
                                    [](const AuxState* a, const AuxState* b) { return a->last_use < b->last_use; });
        free_aux_state(*lru);
        n.states.erase(lru);
    }
    AuxState* S = new AuxState();
    S->key = key;
    S->in_bytes = in_bytes;
    S->out_bytes = out_bytes;
    *st = plan_aux(c, n, *S, B, body);
    if (*st) { free_aux_state(S); return nullptr; }
    S->last_use = ++n.use_clock;
    n.states.push_back(S);
    return S;
}

}  // namespace sdu
