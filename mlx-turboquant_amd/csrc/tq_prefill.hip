// Prefill attention route (tq_prefill.h): eligibility, workspace plan and
// launches; the partials kernel is instantiated for every pair of integer
// key / value widths 2..4.

#include "tq_prefill.h"

namespace tq {

namespace {

// Integer width of a head_dim-128 codec with one codebook (2..4), else 0.
int int_width(const tq_codec* c) {
  if (c->d != 128 || c->split != 128 || !c->centroids_hi || !c->rotation) return 0;
  return c->bits_hi >= 2 && c->bits_hi <= 4 ? c->bits_hi : 0;
}

bool al(const void* p, int n) { return (reinterpret_cast<uintptr_t>(p) & (uintptr_t)(n - 1)) == 0; }

struct Plan {
  int kvrows, nrows, nrows_pad, nd_pad, nbd, nbc, nsplit, bps;
  size_t o_qr, o_dk, o_dv, o_dnk, o_dnv, o_part, total;
};

size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

Plan plan_of(const tq_attn_desc* d) {
  Plan p;
  const int G = d->hq / d->hkv;
  p.kvrows = d->batch * d->hkv;
  p.nrows = d->n_q * G;
  p.nrows_pad = (p.nrows + PREFILL_WAVE_ROWS - 1) / PREFILL_WAVE_ROWS * PREFILL_WAVE_ROWS;
  p.nd_pad = (d->max_sink + d->max_res + 31) / 32 * 32;
  p.nbd = p.nd_pad / 32;
  p.nbc = (d->max_comp + 31) / 32;
  const int nbt = p.nbd + p.nbc;
  const int rows_per_wg = PREFILL_WAVE_ROWS * PREFILL_WAVES;
  const int ny = (p.nrows_pad + rows_per_wg - 1) / rows_per_wg;
  const int64_t base = (int64_t)ny * p.kvrows;
  int ns = (int)std::min<int64_t>((PREFILL_TARGET_WG + base - 1) / base, std::max(1, nbt / 4));
  ns = std::max(ns, 1);
  p.bps = (nbt + ns - 1) / ns;
  p.nsplit = p.bps > 0 ? (nbt + p.bps - 1) / p.bps : 1;
  if (p.bps == 0) p.bps = 1;
  size_t o = 0;
  p.o_qr = o; o = up256(o + (size_t)p.kvrows * p.nrows_pad * 128 * 4);
  p.o_dk = o; o = up256(o + (size_t)p.kvrows * p.nd_pad * 2 * 128 * 2);
  p.o_dv = o; o = up256(o + (size_t)p.kvrows * p.nd_pad * 2 * 128 * 2);
  p.o_dnk = o; o = up256(o + (size_t)p.kvrows * p.nd_pad * 4);
  p.o_dnv = o; o = up256(o + (size_t)p.kvrows * p.nd_pad * 4);
  p.o_part = o; o = up256(o + (size_t)p.nsplit * p.kvrows * p.nrows_pad * PREFILL_PART_FLOATS * 4);
  p.total = o;
  return p;
}

template <int KB, int VB>
void launch_kb_vb(const PrefillArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((pf::prefill_kernel<KB, VB>), grid, dim3(pf::PT), 0, s, a);
}

template <int KB>
int launch_kb(const PrefillArgs& a, int vb, dim3 grid, hipStream_t s) {
  switch (vb) {
    case 2: launch_kb_vb<KB, 2>(a, grid, s); return 0;
    case 3: launch_kb_vb<KB, 3>(a, grid, s); return 0;
    case 4: launch_kb_vb<KB, 4>(a, grid, s); return 0;
  }
  return -1;
}

}  // namespace

// Integer key / value widths 2..4 at head_dim 128, n_q > 1 query tokens, no
// sketch; code rows read as dwords (key rows, 3- and 4-bit value rows) or
// 16-bit words (2-bit value rows), norms as dwords.
bool prefill_eligible(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d) {
  if (!kc || !vc || !d || d->n_q <= 1 || d->qjl || (d->flags & TQ_ATTN_GENERAL)) return false;
  if (d->hkv <= 0 || d->hq % d->hkv) return false;
  const int kb = int_width(kc), vb = int_width(vc);
  if (!kb || !vb) return false;
  if (!al(kc->rotation, 16) || !al(vc->rotation, 16)) return false;  // read as float4
  if (d->max_comp > 0) {
    const tq_store& ks = d->kstore;
    const tq_store& vs = d->vstore;
    const int va = vb == 2 ? 2 : 4;
    if (!al(ks.codes_hi, 4) || ks.hi_head_stride % 4 || !al(vs.codes_hi, va) || vs.hi_head_stride % va) return false;
    if (!al(ks.norms, 4) || !al(vs.norms, 4)) return false;
  }
  const Plan p = plan_of(d);
  const int ny = (p.nrows_pad + PREFILL_WAVE_ROWS * PREFILL_WAVES - 1) / (PREFILL_WAVE_ROWS * PREFILL_WAVES);
  if (ny > 65535 || p.kvrows > 65535 || (int64_t)p.nrows_pad / 32 > 65535 || p.nd_pad / 32 > 65535) return false;
  return true;
}

size_t prefill_workspace(const tq_attn_desc* d) {
  if (!d || d->hkv <= 0 || d->hq % d->hkv || d->n_q <= 1) return 0;
  return plan_of(d).total;
}

int prefill_run(const tq_codec* kc, const tq_codec* vc, const tq_attn_desc* d, void* workspace, hipStream_t s) {
  const Plan p = plan_of(d);
  PrefillArgs a;
  a.batch = d->batch;
  a.hq = d->hq;
  a.hkv = d->hkv;
  a.G = d->hq / d->hkv;
  a.n_q = d->n_q;
  a.kvrows = p.kvrows;
  a.nrows = p.nrows;
  a.nrows_pad = p.nrows_pad;
  a.nd_pad = p.nd_pad;
  a.nbd = p.nbd;
  a.nbc = p.nbc;
  a.nsplit = p.nsplit;
  a.bps = p.bps;
  a.max_comp = d->max_comp;
  a.max_sink = d->max_sink;
  a.max_res = d->max_res;
  a.comp_len = d->comp_len;
  a.sink_len = d->sink_len;
  a.res_len = d->res_len;
  a.res_start = d->res_start;
  a.res_start0 = d->res_start0;
  a.res_cap = d->res_cap;
  a.kc = d->kstore.codes_hi;
  a.k_hs = d->kstore.hi_head_stride;
  a.vc = d->vstore.codes_hi;
  a.v_hs = d->vstore.hi_head_stride;
  a.kn = d->kstore.norms;
  a.kn_hs = d->kstore.norm_head_stride;
  a.vn = d->vstore.norms;
  a.vn_hs = d->vstore.norm_head_stride;
  a.kcen = kc->centroids_hi;
  a.vcen = vc->centroids_hi;
  a.sink_k = d->sink_k;
  a.sink_v = d->sink_v;
  a.sink_hs = d->sink_head_stride;
  a.res_k = d->res_k;
  a.res_v = d->res_v;
  a.res_hs = d->res_head_stride;
  a.kv_dtype = d->kv_dtype;
  a.q = d->q;
  a.q_dtype = d->q_dtype;
  a.rk = kc->rotation;
  a.rv = vc->rotation;
  a.scale = d->scale;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  a.qr = reinterpret_cast<float*>(ws + p.o_qr);
  a.dk = reinterpret_cast<uint16_t*>(ws + p.o_dk);
  a.dv = reinterpret_cast<uint16_t*>(ws + p.o_dv);
  a.dnk = reinterpret_cast<float*>(ws + p.o_dnk);
  a.dnv = reinterpret_cast<float*>(ws + p.o_dnv);
  a.part = reinterpret_cast<float*>(ws + p.o_part);
  a.out = d->out;

  const int gx = std::max(p.nrows_pad, p.nd_pad) / 32;
  hipLaunchKernelGGL(pf::prefill_prep_kernel, dim3(gx, 3, p.kvrows), dim3(256), 0, s, a);
  const int rows_per_wg = PREFILL_WAVE_ROWS * PREFILL_WAVES;
  const dim3 grid(p.nsplit, (p.nrows_pad + rows_per_wg - 1) / rows_per_wg, p.kvrows);
  int rc = -1;
  switch (int_width(kc)) {
    case 2: rc = launch_kb<2>(a, int_width(vc), grid, s); break;
    case 3: rc = launch_kb<3>(a, int_width(vc), grid, s); break;
    case 4: rc = launch_kb<4>(a, int_width(vc), grid, s); break;
  }
  if (rc) return set_error(TQ_ERR_UNSUPPORTED, "prefill: widths K%d / V%d", kc->bits_hi, vc->bits_hi);
  hipLaunchKernelGGL(pf::prefill_merge_kernel, dim3((p.nrows + 15) / 16, p.kvrows), dim3(256), 0, s, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(TQ_ERR_LAUNCH, "prefill attention launch: %s", hipGetErrorString(e));
  return TQ_OK;
}

}  // namespace tq
