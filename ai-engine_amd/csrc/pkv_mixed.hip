// pkv_mixed.hip -- a layer's mixed batch in one launch (gfx950): the
// chunked-prefill workgroups of the prefilling sequences and the decode
// workgroups of the decoding sequences share one grid.
//
// An engine step attends, per layer, the prompt chunks of some sequences
// (Transformer::prefill_seq, crates/ai-engine-candle/src/paged/
// transformer.rs:139-196) and the single new token of all others
// (decode_step, transformer.rs:271-292).  Launched one after the other, the
// prefill (MFMA- and issue-bound on short chunks) and the decode (HBM-bound)
// each leave the other's resource idle, and a HIP graph runs its branches on
// one hardware queue, so two streams do not overlap them either.  Here each
// CU holds workgroups of both kinds at once.
//
// Grid: the prefill workgroups first, then the decode workgroups, each part
// padded to a multiple of kXcd so that a workgroup's virtual block index
// keeps its XCD (the hardware deals workgroups out round-robin; prefill's
// XCD-affine mapping relies on it).  The prefill workgroups are the long
// ones (a chain of key tiles each), so they are dispatched at once and the
// short decode workgroups stream through the slots they leave free (cfg2:
// two prefill workgroups and one decode workgroup per CU), then through all
// slots once the prefill drains.  Spreading the decode groups evenly among
// the prefill groups was measured slower than two separate launches: the
// last prefill workgroups then start only after most of the decode.  A
// workgroup runs the unchanged prefill or decode body, so every output and
// every stored row is bit-identical to the two separate launches.  The
// split-context merges (decode; prefill when it splits) follow as their own
// launches, their partials in disjoint parts of the pool workspace.
//
// LDS: the two bodies' LDS overlap in one union (a workgroup runs one body);
// registers are the larger body's.  Built for 16-bit pools, head_dim 64 and
// 128 and GQA ratios 4 and 8 (the shapes of Llama, Mistral and TinyLlama
// class models; f16 at head_dim 128 only for GQA 8); other shapes run the
// two launches in sequence.
#include "pkv_decode_dev.h"
#include "pkv_prefill_dev.h"

namespace pkv {
namespace {

static_assert(kPT == kWavesPerBlock * kWave, "prefill and decode workgroups must match");

template <int DT, int HD, int R>
union alignas(16) MixedSmem {
  char pre[2 * PCfg<DT, HD, R>::STAGE];
  DecodeSmem<DT, HD, R> dec;
};

template <int DT, int HD, int R, bool FUSED>
__global__ void __launch_bounds__(kPT)
    mixed_kernel(PrefillKArgs pa, DecodeKArgs da, int pgroups) {
  __shared__ MixedSmem<DT, HD, R> sm;
  const int gi = blockIdx.x / kXcd;
  const int x = blockIdx.x % kXcd;
  if (gi >= pgroups)
    decode_body<DT, HD, R, false, false>(da, (gi - pgroups) * kXcd + x, sm.dec);
  else
    prefill_body<DT, HD, R, FUSED, false>(pa, gi * kXcd + x, sm.pre);
}

template <int DT, int HD, int R, bool FUSED>
hipError_t mixed_t(PrefillKArgs pk, const DecodeKArgs& dk, long long ditems, hipStream_t s) {
  const long long pgrid = prefill_grid<DT, HD, R>(pk);
  const long long dgrid = (ditems + kWavesPerBlock - 1) / kWavesPerBlock;
  const long long pg = (pgrid + kXcd - 1) / kXcd, dg = (dgrid + kXcd - 1) / kXcd;
  if (!grid_fits((pg + dg) * kXcd, kPT)) return hipErrorInvalidValue;
  if (pg + dg == 0) return hipSuccess;
  mixed_kernel<DT, HD, R, FUSED>
      <<<(unsigned)((pg + dg) * kXcd), kPT, 0, s>>>(pk, dk, (int)pg);
  return hipGetLastError();
}

template <int DT, int HD, int R>
hipError_t mixed_f(const PrefillKArgs& pk, const DecodeKArgs& dk, long long ditems,
                   hipStream_t s) {
  return pk.k_new ? mixed_t<DT, HD, R, true>(pk, dk, ditems, s)
                  : mixed_t<DT, HD, R, false>(pk, dk, ditems, s);
}

// f16 pools of head_dim 128 at GQA 4 are left out: the combined kernel
// would need more than 256 registers (one wave per SIMD).
constexpr bool mixed_built(int dt, int hd, int r) {
  return (r == 4 || r == 8) && (hd == 64 || hd == 128) && (dt == PKV_F16 || dt == PKV_BF16) &&
         !(dt == PKV_F16 && hd == 128 && r == 4);
}

template <int DT, int HD>
hipError_t mixed_r(int R, const PrefillKArgs& pk, const DecodeKArgs& dk, long long ditems,
                   hipStream_t s) {
  if (R == 8) return mixed_f<DT, HD, 8>(pk, dk, ditems, s);
  if constexpr (mixed_built(DT, HD, 4)) return mixed_f<DT, HD, 4>(pk, dk, ditems, s);
  return hipErrorNotSupported;
}

template <int DT>
hipError_t mixed_hd(int HD, int R, const PrefillKArgs& pk, const DecodeKArgs& dk,
                    long long ditems, hipStream_t s) {
  return HD == 64 ? mixed_r<DT, 64>(R, pk, dk, ditems, s) : mixed_r<DT, 128>(R, pk, dk, ditems, s);
}

}  // namespace

bool mixed_supported(const pkv_pool* p, int n_head, bool rope) {
  // block_size >= 16: the decode body here is the one with uniform block ids
  if (rope || n_head <= 0 || n_head % p->n_kv_head || p->block_size < 16) return false;
  return mixed_built(p->dtype, p->head_dim, n_head / p->n_kv_head);
}

hipError_t launch_mixed(const pkv_pool* p, int layer, const PrefillArgs& pa,
                        const DecodeArgs& da, char* decode_partials, char* prefill_partials,
                        hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  if (pa.n_head != da.n_head || !mixed_supported(p, da.n_head, da.rope_cos != nullptr))
    return hipErrorNotSupported;
  long long ditems = 0;
  const DecodeKArgs dk = decode_kargs(p, layer, da, decode_partials, 0, &ditems);
  const PrefillKArgs pk = prefill_kargs(p, layer, pa, prefill_partials);
  const int R = da.n_head / p->n_kv_head;
  hipError_t e = hipSuccess;
  if (ev_begin && (e = hipEventRecord(ev_begin, stream)) != hipSuccess) return e;
  e = p->dtype == PKV_F16 ? mixed_hd<PKV_F16>(p->head_dim, R, pk, dk, ditems, stream)
                          : mixed_hd<PKV_BF16>(p->head_dim, R, pk, dk, ditems, stream);
  if (e != hipSuccess) return e;
  if (ev_end && (e = hipEventRecord(ev_end, stream)) != hipSuccess) return e;
  if ((e = launch_decode_merge(p, dk, stream)) != hipSuccess) return e;
  return launch_prefill_merge(p, pk, stream);
}

}  // namespace pkv
