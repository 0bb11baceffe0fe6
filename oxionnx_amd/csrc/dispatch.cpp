// Node-level dispatch: the provider's counterpart of oxionnx-cuda's
// try_cuda_dispatch / try_cuda_dispatch_resident (oxionnx-cuda/src/lib.rs:354-960).
// A node arrives with its ONNX op type, attributes and operands (host tensors
// or resident device tensors); the provider either claims it (OHIP_OK, outputs
// returned on the host or kept on the device), declines it (OHIP_DECLINED: the
// caller runs its CPU operator, which also reports malformed-model errors), or
// fails (< 0).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ohip.h"
#include "internal.hpp"

int ohip_dtensor_alias_internal(const ohip_dtensor* src, int rank, const int64_t* shape, ohip_dtensor** out);
int ohip_dtensor_view_internal(const ohip_dtensor* src, int rank, const int64_t* shape, size_t byte_offset,
                               ohip_dtensor** out);
int ohip_const_operand_internal(ohip_ctx* ctx, const char* name, const char* label, int dtype, const void* host,
                                size_t bytes, const void** dev);
int ohip_dtensor_set_nhwc_internal(ohip_dtensor* t, int64_t pitch);
int64_t ohip_dtensor_pitch_internal(const ohip_dtensor* t);
int ohip_dtensor_view_nhwc_internal(const ohip_dtensor* src, int64_t c0, int64_t cn, ohip_dtensor** out);
int ohip_dtensor_to_nchw_internal(ohip_ctx* ctx, const ohip_dtensor* t, void* dst);
int ohip_hip_error_internal(hipError_t e, const char* what);
int ohip_conv_halo_splits_internal(ohip_ctx* ctx, const ohip_conv_desc* d);
int ohip_conv_fewco_internal(const ohip_conv_desc* d);

namespace {

thread_local std::string t_err;

int decline(const std::string& why) {
  t_err = why;
  return OHIP_DECLINED;
}

// The size gate prices a transfer: an operand that is already a resident
// device tensor skips it (skips_size_threshold,
// oxionnx-gpu/src/context/activation.rs:248-250), since declining would read
// it back for a CPU kernel instead.
bool any_resident(const ohip_node* nd) {
  for (int i = 0; i < nd->n_inputs; ++i)
    if (nd->inputs[i].device) return true;
  return false;
}

// ------------------------------------------------------------------ attributes
const ohip_attr* find_attr(const ohip_node* n, const char* name) {
  for (int i = 0; i < n->n_attrs; ++i)
    if (n->attrs[i].name && std::strcmp(n->attrs[i].name, name) == 0) return &n->attrs[i];
  return nullptr;
}
int64_t attr_i(const ohip_node* n, const char* name, int64_t dflt) {
  const ohip_attr* a = find_attr(n, name);
  return a && a->kind == OHIP_ATTR_INT ? a->i : dflt;
}
float attr_f(const ohip_node* n, const char* name, float dflt) {
  const ohip_attr* a = find_attr(n, name);
  if (!a) return dflt;
  if (a->kind == OHIP_ATTR_FLOAT) return a->f;
  if (a->kind == OHIP_ATTR_INT) return (float)a->i;
  return dflt;
}
std::vector<int64_t> attr_ints(const ohip_node* n, const char* name) {
  const ohip_attr* a = find_attr(n, name);
  if (!a || a->kind != OHIP_ATTR_INTS || !a->ints) return {};
  return std::vector<int64_t>(a->ints, a->ints + a->n_ints);
}
std::string attr_s(const ohip_node* n, const char* name) {
  const ohip_attr* a = find_attr(n, name);
  return a && a->kind == OHIP_ATTR_STRING && a->s ? std::string(a->s) : std::string();
}

// ------------------------------------------------------------------ operands
const ohip_tensor* input(const ohip_node* n, int i) {
  if (i >= n->n_inputs) return nullptr;
  const ohip_tensor* t = &n->inputs[i];
  if (!t->data && !t->device) return nullptr;  // an absent optional input
  return t;
}
int64_t numel(const ohip_tensor* t) {
  int64_t e = 1;
  for (int i = 0; i < t->rank; ++i) e *= t->shape[i];
  return e;
}
int ebytes(int dt) {
  switch (dt) {
    case OHIP_F32: case OHIP_I32: return 4;
    case OHIP_F16: case OHIP_BF16: return 2;
    case OHIP_U8: case OHIP_I8: return 1;
    default: return 0;
  }
}
bool host_only(const ohip_tensor* t) { return t && t->data; }

// Element i of a host tensor as double (integers exact).
double host_at(const ohip_tensor* t, int64_t i) {
  switch (t->dtype) {
    case OHIP_F32: return static_cast<const float*>(t->data)[i];
    case OHIP_I32: return static_cast<const int32_t*>(t->data)[i];
    case OHIP_U8: return static_cast<const uint8_t*>(t->data)[i];
    case OHIP_I8: return static_cast<const int8_t*>(t->data)[i];
    case OHIP_F16: {
      uint16_t h = static_cast<const uint16_t*>(t->data)[i];
      // exact f16 -> f32 widening
      uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff, x;
      if (e == 0) {
        if (!m) x = s;
        else {
          int k = -1;
          do { m <<= 1; ++k; } while (!(m & 0x400u));
          x = s | ((uint32_t)(112 - k) << 23) | ((m & 0x3ffu) << 13);
        }
      } else if (e == 31) x = s | 0x7f800000u | (m << 13);
      else x = s | ((e + 112) << 23) | (m << 13);
      float f;
      std::memcpy(&f, &x, 4);
      return f;
    }
    case OHIP_BF16: {
      uint32_t x = (uint32_t) static_cast<const uint16_t*>(t->data)[i] << 16;
      float f;
      std::memcpy(&f, &x, 4);
      return f;
    }
    default: return NAN;
  }
}

// Store v as element idx of a dtype buffer (f16 / bf16 round to nearest even).
void put_elem(int dt, void* buf, int64_t idx, double v) {
  const float f = (float)v;
  if (dt == OHIP_F32) {
    std::memcpy(static_cast<char*>(buf) + idx * 4, &f, 4);
  } else if (dt == OHIP_F16) {
    const _Float16 h = (_Float16)f;
    std::memcpy(static_cast<char*>(buf) + idx * 2, &h, 2);
  } else if (dt == OHIP_BF16) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint16_t h = (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u)
                                                                     : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16));
    std::memcpy(static_cast<char*>(buf) + idx * 2, &h, 2);
  }
}

// round half to even, the lane_to_i32 rule (quant_ops/mod.rs:74-92)
bool lane_int(double v, int32_t* out) {
  if (!std::isfinite(v)) return false;
  double r = std::nearbyint(v);
  if (r < INT32_MIN || r > INT32_MAX) return false;
  *out = (int32_t)r;
  return true;
}

// Quantised lanes -> bytes.  Picks u8 when every lane is in 0..255, else i8
// when every lane is in -128..127; anything else is declined.
bool to_bytes(const ohip_tensor* t, std::vector<uint8_t>& out, int* dt) {
  const int64_t n = numel(t);
  out.resize((size_t)n);
  if (t->dtype == OHIP_U8 || t->dtype == OHIP_I8) {
    std::memcpy(out.data(), t->data, (size_t)n);
    *dt = t->dtype;
    return true;
  }
  int32_t lo = INT32_MAX, hi = INT32_MIN;
  std::vector<int32_t> v((size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    if (!lane_int(host_at(t, i), &v[(size_t)i])) return false;
    lo = std::min(lo, v[(size_t)i]);
    hi = std::max(hi, v[(size_t)i]);
  }
  if (n == 0) lo = hi = 0;
  if (lo >= 0 && hi <= 255) *dt = OHIP_U8;
  else if (lo >= -128 && hi <= 127) *dt = OHIP_I8;
  else return false;
  for (int64_t i = 0; i < n; ++i) out[(size_t)i] = (uint8_t)(v[(size_t)i] & 0xff);
  return true;
}

// zero_point_lanes (quant_ops/mod.rs:121-127): absent or empty -> [0].
bool zp_lanes(const ohip_tensor* t, std::vector<int32_t>& out) {
  out.clear();
  if (!t || numel(t) == 0) {
    out.push_back(0);
    return true;
  }
  if (!host_only(t)) return false;
  for (int64_t i = 0; i < numel(t); ++i) {
    int32_t v;
    if (!lane_int(host_at(t, i), &v)) return false;
    out.push_back(v);
  }
  return true;
}

// scale_input (quant_ops/mod.rs:100-118): first element, finite, non-zero.
bool scale_first(const ohip_tensor* t, float* s) {
  if (!host_only(t) || numel(t) == 0) return false;
  double v = host_at(t, 0);
  if (!std::isfinite(v) || v == 0.0) return false;
  *s = (float)v;
  return true;
}

// SatRange::infer / for_dtype (quant_ops/mod.rs:188-221).
void sat_range(const ohip_tensor* yzp_t, const std::vector<int32_t>& yzp, const std::vector<int32_t>& xzp,
               int32_t* lo, int32_t* hi) {
  if (yzp_t && yzp_t->declared_dtype == OHIP_U8) { *lo = 0; *hi = 255; return; }
  if (yzp_t && yzp_t->declared_dtype == OHIP_I8) { *lo = -128; *hi = 127; return; }
  for (const auto* lanes : {&yzp, &xzp}) {
    for (int32_t v : *lanes) if (v > 127) { *lo = 0; *hi = 255; return; }
    for (int32_t v : *lanes) if (v < 0) { *lo = -128; *hi = 127; return; }
  }
  *lo = -128;
  *hi = 255;
}

// ------------------------------------------------------------------ staging
struct Stage {
  ohip_ctx* ctx;
  std::vector<void*> bufs;
  explicit Stage(ohip_ctx* c) : ctx(c) {}
  ~Stage() {
    for (void* p : bufs) ohip_free(ctx, p);
  }
  void* alloc(size_t bytes) {
    void* p = nullptr;
    if (ohip_malloc(ctx, bytes ? bytes : 16, &p) != OHIP_OK) return nullptr;
    bufs.push_back(p);
    return p;
  }
  // A host initializer operand (already converted to `host` / `bytes`, in
  // dtype `dt`): the context's session-lifetime device copy.  Any other host
  // tensor is copied for this call.
  const void* cached(const ohip_tensor* t, const char* label, int dt, const void* host, size_t bytes) {
    if (t->device) return ohip_dtensor_ptr(t->device);
    if (t->is_initializer && t->name && *t->name) {
      const void* d = nullptr;
      if (ohip_const_operand_internal(ctx, t->name, label, dt, host, bytes, &d) != OHIP_OK) return nullptr;
      return d;
    }
    return operand(t, host, bytes);
  }
  // A device copy of a host tensor (or the resident pointer itself).
  const void* operand(const ohip_tensor* t, const void* host_override = nullptr, size_t bytes = 0) {
    if (t->device && !host_override) return ohip_dtensor_ptr(t->device);
    const void* src = host_override ? host_override : t->data;
    size_t nb = host_override ? bytes : (size_t)numel(t) * ebytes(t->dtype);
    void* d = alloc(nb);
    if (!d || ohip_memcpy_h2d(ctx, d, src, nb) != OHIP_OK) return nullptr;
    return d;
  }
};

// OHIP_NHWC=0 keeps every resident convolution output NCHW (a measurement
// switch)
bool nhwc_residency() {
  static const bool v = [] {
    const char* e = std::getenv("OHIP_NHWC");
    return !(e && e[0] == '0');
  }();
  return v;
}

void set_out(ohip_output* o, int dtype, const std::vector<int64_t>& shape) {
  std::memset(o, 0, sizeof(*o));
  o->dtype = dtype;
  o->rank = (int)shape.size();
  for (size_t i = 0; i < shape.size() && i < 8; ++i) o->shape[i] = shape[i];
}

int finish_output(ohip_ctx* ctx, Stage& st, int placement, ohip_output* o, void* dev, size_t bytes, int dev_dtype) {
  if (placement == OHIP_PLACE_DEVICE) {
    ohip_dtensor* t = nullptr;
    int rc = ohip_dtensor_wrap(ctx, dev, dev_dtype, o->rank, o->shape, &t);
    if (rc) return rc;
    st.bufs.erase(std::remove(st.bufs.begin(), st.bufs.end(), dev), st.bufs.end());  // now owned by t
    o->device = t;
    return OHIP_OK;
  }
  o->data = std::malloc(bytes ? bytes : 1);
  if (!o->data) return OHIP_E_NOMEM;
  return ohip_memcpy_d2h(ctx, o->data, dev, bytes);
}

// ------------------------------------------------------------------ Conv geometry
struct Geo {
  int64_t n, c, h, w, cout, kh, kw, group;
  int64_t sh, sw, dh, dw, pt, pl, pb, pr, oh, ow;
  bool rank1;
};

// ConvGeometry::from_attrs (registry/conv_ops/conv.rs:38-121) and
// resolve_pads / same_pad_split (conv/spatial.rs:204-257), rank 1 and 2.
bool conv_geometry(const ohip_node* nd, const ohip_tensor* x, const ohip_tensor* w, Geo* g, std::string* why) {
  if (x->rank != w->rank || (x->rank != 3 && x->rank != 4)) { *why = "Conv: only rank 1 and 2 spatial"; return false; }
  g->rank1 = x->rank == 3;
  g->n = x->shape[0];
  g->c = x->shape[1];
  g->h = g->rank1 ? 1 : x->shape[2];
  g->w = x->shape[x->rank - 1];
  g->cout = w->shape[0];
  g->kh = g->rank1 ? 1 : w->shape[2];
  g->kw = w->shape[w->rank - 1];
  g->group = attr_i(nd, "group", 1);
  if (g->group <= 0 || w->shape[1] * g->group != g->c || g->cout % g->group) { *why = "Conv: bad group"; return false; }
  const int sr = g->rank1 ? 1 : 2;
  auto strides = attr_ints(nd, "strides"), dil = attr_ints(nd, "dilations"), pads = attr_ints(nd, "pads");
  auto ks = attr_ints(nd, "kernel_shape");
  if (!ks.empty()) {
    if ((int)ks.size() != sr || ks.back() != g->kw || (sr == 2 && ks[0] != g->kh)) {
      *why = "Conv: kernel_shape disagrees with W";
      return false;
    }
  }
  if (strides.empty()) strides.assign(sr, 1);
  if (dil.empty()) dil.assign(sr, 1);
  if (pads.empty()) pads.assign(2 * sr, 0);
  if ((int)strides.size() != sr || (int)dil.size() != sr || (int)pads.size() != 2 * sr) {
    *why = "Conv: attribute rank mismatch";
    return false;
  }
  for (auto v : strides) if (v <= 0) { *why = "Conv: stride"; return false; }
  for (auto v : dil) if (v <= 0) { *why = "Conv: dilation"; return false; }
  for (auto v : pads) if (v < 0) { *why = "Conv: negative pad"; return false; }
  g->sh = sr == 2 ? strides[0] : 1;
  g->sw = strides.back();
  g->dh = sr == 2 ? dil[0] : 1;
  g->dw = dil.back();
  int64_t pt = sr == 2 ? pads[0] : 0, pl = sr == 2 ? pads[1] : pads[0];
  int64_t pb = sr == 2 ? pads[2] : 0, pr = sr == 2 ? pads[3] : pads[1];
  std::string ap = attr_s(nd, "auto_pad");
  if (ap == "VALID") pt = pl = pb = pr = 0;
  else if (ap == "SAME_UPPER" || ap == "SAME_LOWER") {
    auto split = [&](int64_t in, int64_t k, int64_t s, int64_t d, int64_t* b, int64_t* e) {
      int64_t out = (in + s - 1) / s, eff = (k - 1) * d + 1;
      int64_t need = std::max<int64_t>(0, (out - 1) * s + eff - in), half = need / 2;
      if (ap == "SAME_LOWER") { *b = need - half; *e = half; } else { *b = half; *e = need - half; }
    };
    if (sr == 2) split(g->h, g->kh, g->sh, g->dh, &pt, &pb);
    split(g->w, g->kw, g->sw, g->dw, &pl, &pr);
  } else if (!(ap.empty() || ap == "NOTSET")) {
    *why = "Conv: unknown auto_pad";
    return false;
  }
  g->pt = pt; g->pl = pl; g->pb = pb; g->pr = pr;
  g->oh = ohip_conv_out_dim(g->h, pt, pb, g->kh, g->dh, g->sh);
  g->ow = ohip_conv_out_dim(g->w, pl, pr, g->kw, g->dw, g->sw);
  if (g->oh < 0 || g->ow < 0) { *why = "Conv: output extent"; return false; }
  return true;
}

std::vector<int64_t> conv_out_shape(const Geo& g) {
  if (g.rank1) return {g.n, g.cout, g.ow};
  return {g.n, g.cout, g.oh, g.ow};
}

// apply_fused_activation's attribute contract (registry/conv_ops/conv.rs:124-156).
void fused_act(const ohip_node* nd, int* act, float* lo, float* hi) {
  std::string a = attr_s(nd, "activation");
  *act = OHIP_ACT_NONE;
  *lo = 0.0f;
  *hi = 0.0f;
  if (a == "relu") *act = OHIP_ACT_RELU;
  else if (a == "leaky_relu") {  // this provider's Conv + LeakyRelu fusion
    *act = OHIP_ACT_LEAKY_RELU;
    *lo = attr_f(nd, "activation_alpha", 0.01f);
  } else if (a == "clip") {
    *act = OHIP_ACT_CLIP;
    *lo = attr_f(nd, "activation_min", -INFINITY);
    *hi = attr_f(nd, "activation_max", INFINITY);
  }
}

std::string wkey_name(const ohip_tensor* t) { return t->name ? std::string(t->name) : std::string(); }

// ------------------------------------------------------------------ float Conv
bool bcast_plan(const int64_t* as, int ra, const int64_t* bs, int rb, ohip::BcastPlan* p, std::vector<int64_t>* oshape,
                int64_t* n_out);
const void* float_operand(Stage& st, const ohip_tensor* t, int dt);

// with_norm: this provider's fused Conv -> OxiInstanceNorm node
// (OhipConvInstanceNorm): inputs 0-2 are the Conv's, inputs 3 / 4 the
// optional AdaIN modulation rows (resident [N, S], as the fused
// OxiInstanceNorm takes them), attributes the Conv's plus "epsilon",
// "scale_offset", "bias_offset" and "norm_activation" ("relu" or empty).
int do_conv(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out, bool with_norm = false) {
  const ohip_tensor *x = input(nd, 0), *w = input(nd, 1), *b = input(nd, 2);
  if (!x || !w) return decline("Conv: missing input");
  if (!host_only(w) || (b && !host_only(b))) return decline("Conv: filter / bias must be host tensors");
  const int dt = x->dtype;
  if (dt != OHIP_F32 && dt != OHIP_F16 && dt != OHIP_BF16) return decline("Conv: dtype");
  Geo g;
  std::string why;
  if (!conv_geometry(nd, x, w, &g, &why)) return decline(why);
  const int64_t cg = g.c / g.group;
  ohip_tuning tun;
  ohip_get_tuning(ctx, &tun);
  // the fused node has no host counterpart to fall back to: it always runs here
  if (!with_norm && !any_resident(nd) && !ohip_conv_admits(&tun, g.cout, cg * g.kh * g.kw, g.n * g.oh * g.ow))
    return decline("Conv: below conv_min_mac");
  // a resident NHWC input reaches here only where the halo-patch path reads
  // it in place (takes_nhwc)
  const bool x_nhwc = x->device && ohip_dtensor_layout(x->device) == OHIP_NHWC;
  if (x_nhwc && ohip_dtensor_pitch_internal(x->device) != g.c) return decline("Conv: NHWC pixel pitch");

  std::string name = wkey_name(w), label = "Conv.W";
  ohip_weight_key key{name.c_str(), label.c_str()};
  const bool cache = w->is_initializer && !name.empty();
  ohip_weight* wt = nullptr;
  int rc = ohip_weight_conv(ctx, cache ? &key : nullptr, w->dtype, w->data, g.cout, cg, g.kh, g.kw, dt, &wt);
  if (rc) return rc;
  Stage st(ctx);
  const void* xd = st.operand(x);
  const void* bd = nullptr;
  std::vector<char> bconv;
  if (b) {
    if (numel(b) != g.cout) {
      if (!cache) ohip_weight_release(wt);
      return decline("Conv: bias length");
    }
    if (b->dtype != dt) {  // e.g. f32 bias lanes on a typed conv: round once (RNE)
      bconv.resize((size_t)g.cout * ebytes(dt));
      for (int64_t i = 0; i < g.cout; ++i) put_elem(dt, bconv.data(), i, host_at(b, i));
      bd = st.cached(b, "Conv.B", dt, bconv.data(), bconv.size());
    } else {
      bd = st.cached(b, "Conv.B", dt, b->data, (size_t)numel(b) * ebytes(dt));
    }
  }
  const auto oshape = conv_out_shape(g);
  const size_t obytes = (size_t)(g.n * g.cout * g.oh * g.ow) * ebytes(dt);
  void* yd = st.alloc(obytes);
  if (!xd || !yd || (b && !bd)) { if (!cache) ohip_weight_release(wt); return OHIP_E_NOMEM; }
  // a fused residual (input 5) of another shape is broadcast by the binary
  // kernel after the fused pair, which indexes the pair's output as NCHW
  const ohip_tensor* res_in = with_norm && nd->n_inputs > 5 ? input(nd, 5) : nullptr;
  const bool res_bcast = res_in && !(res_in->rank == (int)oshape.size() &&
                                     std::equal(oshape.begin(), oshape.end(), res_in->shape));
  // a session layout hint: every consumer of this output reads NHWC in place
  const bool y_nhwc = placement == OHIP_PLACE_DEVICE && attr_i(nd, "out_nhwc", 0) == 1 && g.group == 1 &&
                      !g.rank1 && g.cout % (16 / ebytes(dt)) == 0 && (!with_norm || g.cout % 8 == 0) &&
                      !res_bcast;
  ohip_conv_desc d{g.n, g.c, g.h, g.w, g.cout, g.kh, g.kw, g.group, g.sh, g.sw, g.dh, g.dw, g.pt, g.pl, g.pb, g.pr,
                   dt, x_nhwc ? OHIP_NHWC : OHIP_NCHW, y_nhwc ? OHIP_NHWC : OHIP_NCHW, 0, 0.0f, 0.0f,
                   OHIP_PAD_ZEROS};
  fused_act(nd, &d.act, &d.act_lo, &d.act_hi);
  // this provider's Pad -> Conv fusion: the pads are a reflect / edge Pad's
  {
    const std::string pm = attr_s(nd, "pad_mode");
    if (pm == "reflect") d.pad_mode = OHIP_PAD_REFLECT;
    else if (pm == "edge") d.pad_mode = OHIP_PAD_EDGE;
    else if (!pm.empty() && pm != "constant") {
      if (!cache) ohip_weight_release(wt);
      return decline("Conv: pad_mode");
    }
  }
  if (with_norm) {
    ohip_norm_desc nm{};
    nm.epsilon = attr_f(nd, "epsilon", 1e-5f);
    const ohip_tensor *gm = nd->n_inputs > 3 ? input(nd, 3) : nullptr, *bt = nd->n_inputs > 4 ? input(nd, 4) : nullptr;
    if (gm || bt) {
      if (!gm || !bt || !gm->device || !bt->device || gm->dtype != dt || bt->dtype != dt || gm->rank != 2 ||
          bt->rank != 2 || gm->shape[0] != g.n || bt->shape[0] != g.n || gm->shape[1] != bt->shape[1]) {
        if (!cache) ohip_weight_release(wt);
        return decline("ConvInstanceNorm: modulation operands must be resident [N, S] rows of the input's dtype");
      }
      const int64_t so = attr_i(nd, "scale_offset", 0), bo = attr_i(nd, "bias_offset", 0), S = gm->shape[1];
      if (so < 0 || bo < 0 || so + g.cout > S || bo + g.cout > S) {
        if (!cache) ohip_weight_release(wt);
        return decline("ConvInstanceNorm: modulation offsets");
      }
      nm.scale = static_cast<const char*>(ohip_dtensor_ptr(gm->device)) + so * ebytes(dt);
      nm.bias = static_cast<const char*>(ohip_dtensor_ptr(bt->device)) + bo * ebytes(dt);
      nm.per_sample = 1;
      nm.stride = S;
      nm.same_type = 1;
    }
    const std::string na = attr_s(nd, "norm_activation");
    if (na == "relu") nm.act = OHIP_ACT_RELU;
    else if (!na.empty()) {
      if (!cache) ohip_weight_release(wt);
      return decline("ConvInstanceNorm: activation");
    }
    // input 5: a fused residual Add (the other operand of an Add that was the
    // norm's only consumer); added in the kernel when it has the output's
    // shape, else broadcast by the binary kernel after the fused pair
    const ohip_tensor* res = nd->n_inputs > 5 ? input(nd, 5) : nullptr;
    if (res) {
      const void* rd = float_operand(st, res, dt);
      if (!rd) {
        if (!cache) ohip_weight_release(wt);
        return decline("ConvInstanceNorm: residual dtype");
      }
      const bool same = res->rank == (int)oshape.size() &&
                        std::equal(oshape.begin(), oshape.end(), res->shape);
      if (same) {
        nm.residual = rd;
        nm.residual_layout = res->device ? ohip_dtensor_layout(res->device) : OHIP_NCHW;
        rc = ohip_conv2d_instnorm(ctx, &d, xd, wt, bd, &nm, yd);
      } else {
        ohip::BcastPlan p{};
        std::vector<int64_t> bshape;
        int64_t n = 0;
        if (!bcast_plan(oshape.data(), (int)oshape.size(), res->shape, res->rank, &p, &bshape, &n)) {
          if (!cache) ohip_weight_release(wt);
          return decline("ConvInstanceNorm: residual shape");
        }
        void* bd2 = st.alloc((size_t)n * ebytes(dt));
        if (!bd2) { if (!cache) ohip_weight_release(wt); return OHIP_E_NOMEM; }
        rc = ohip_conv2d_instnorm(ctx, &d, xd, wt, bd, &nm, yd);
        if (rc == OHIP_OK) {
          hipError_t e = ohip::run_binary(dt, yd, rd, bd2, n, p, false, ohip::BIN_ADD,
                                          (hipStream_t)ohip_ctx_stream(ctx));
          if (e != hipSuccess) rc = ohip_hip_error_internal(e, "node kernel launch");
        }
        if (!cache) ohip_weight_release(wt);
        if (rc) return rc;
        set_out(out, dt, bshape);
        return finish_output(ctx, st, placement, out, bd2, (size_t)n * ebytes(dt), dt);
      }
    } else {
      rc = ohip_conv2d_instnorm(ctx, &d, xd, wt, bd, &nm, yd);
    }
  } else {
    rc = ohip_conv2d(ctx, &d, xd, wt, bd, yd);
  }
  if (!cache) ohip_weight_release(wt);
  if (rc) return rc;
  set_out(out, dt, oshape);
  rc = finish_output(ctx, st, placement, out, yd, obytes, dt);
  if (rc == OHIP_OK && y_nhwc) rc = ohip_dtensor_set_nhwc_internal(out->device, g.cout);
  return rc;
}

// Whether a float conv (or the conv of the fused conv + norm node) reads a
// resident NHWC input in place: ungrouped, on the halo-patch path at this
// geometry.
bool conv_takes_nhwc(ohip_ctx* ctx, const ohip_node* nd) {
  const ohip_tensor *x = input(nd, 0), *w = input(nd, 1);
  if (!x || !w || !x->device || x->rank != 4) return false;
  Geo g;
  std::string why;
  if (!conv_geometry(nd, x, w, &g, &why) || g.group != 1) return false;
  if (ohip_dtensor_pitch_internal(x->device) != g.c) return false;
  ohip_conv_desc d{g.n, g.c, g.h, g.w, g.cout, g.kh, g.kw, g.group, g.sh, g.sw, g.dh, g.dw, g.pt, g.pl, g.pb, g.pr,
                   x->dtype, OHIP_NHWC, OHIP_NCHW, 0, 0.0f, 0.0f, OHIP_PAD_ZEROS};
  const std::string pm = attr_s(nd, "pad_mode");
  if (pm == "reflect") d.pad_mode = OHIP_PAD_REFLECT;
  else if (pm == "edge") d.pad_mode = OHIP_PAD_EDGE;
  // zero padding: the engine's implicit im2col reads the NHWC tensor as it
  // is; a reflect / edge pad is applied in place only by the halo path
  if (d.pad_mode == OHIP_PAD_ZEROS) return true;
  return ohip_conv_halo_splits_internal(ctx, &d) > 0 || ohip_conv_fewco_internal(&d) != 0;
}

// ------------------------------------------------------------------ ConvTranspose
// ConvTransposeGeometry::from_attrs (registry/conv_ops/conv.rs:349-470) with
// derive_transpose_pads (:519-554) and read_output_shape_attr (:490-515),
// rank 2: output_shape (2 or 4 entries) or SAME_* auto_pad fix the target
// extent and the pads are derived from it; otherwise the explicit pads (or
// none for VALID) crop the natural extent.
int do_conv_transpose(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor *x = input(nd, 0), *w = input(nd, 1), *b = input(nd, 2);
  if (!x || !w) return decline("ConvTranspose: missing input");
  if (!host_only(w) || (b && !host_only(b))) return decline("ConvTranspose: filter / bias must be host tensors");
  const int dt = x->dtype;
  if (dt != OHIP_F32 && dt != OHIP_F16 && dt != OHIP_BF16) return decline("ConvTranspose: dtype");
  if (x->rank != 4 || w->rank != 4) return decline("ConvTranspose: only rank 2 spatial");
  if (x->device && ohip_dtensor_layout(x->device) != OHIP_NCHW) return decline("ConvTranspose: resident input layout");
  const int64_t n = x->shape[0], c = x->shape[1], h = x->shape[2], wd = x->shape[3];
  const int64_t coutg = w->shape[1], kh = w->shape[2], kw = w->shape[3];
  const int64_t group = attr_i(nd, "group", 1);
  if (group <= 0 || w->shape[0] != c || c % group) return decline("ConvTranspose: bad group / channels");
  auto strides = attr_ints(nd, "strides"), dil = attr_ints(nd, "dilations"), pads = attr_ints(nd, "pads");
  auto opad = attr_ints(nd, "output_padding"), oshape = attr_ints(nd, "output_shape"), ks = attr_ints(nd, "kernel_shape");
  if (!ks.empty() && (ks.size() != 2 || ks[0] != kh || ks[1] != kw)) return decline("ConvTranspose: kernel_shape");
  if (strides.empty()) strides.assign(2, 1);
  if (dil.empty()) dil.assign(2, 1);
  if (pads.empty()) pads.assign(4, 0);
  if (opad.empty()) opad.assign(2, 0);
  if (strides.size() != 2 || dil.size() != 2 || pads.size() != 4 || opad.size() != 2)
    return decline("ConvTranspose: attribute rank mismatch");
  for (int a = 0; a < 2; ++a)
    if (strides[a] <= 0 || dil[a] <= 0 || opad[a] < 0) return decline("ConvTranspose: stride / dilation / output_padding");
  for (auto v : pads) if (v < 0) return decline("ConvTranspose: negative pad");
  const std::string ap = attr_s(nd, "auto_pad");
  if (!(ap.empty() || ap == "NOTSET" || ap == "VALID" || ap == "SAME_UPPER" || ap == "SAME_LOWER"))
    return decline("ConvTranspose: unknown auto_pad");
  const int64_t in[2] = {h, wd}, kk[2] = {kh, kw};
  bool has_target = false;
  int64_t target[2] = {0, 0};
  if (!oshape.empty()) {
    if (oshape.size() != 2 && oshape.size() != 4) return decline("ConvTranspose: output_shape length");
    target[0] = oshape[oshape.size() - 2];
    target[1] = oshape[oshape.size() - 1];
    if (target[0] < 1 || target[1] < 1) return decline("ConvTranspose: output_shape");
    has_target = true;
  } else if (ap == "SAME_UPPER" || ap == "SAME_LOWER") {
    target[0] = h * strides[0];
    target[1] = wd * strides[1];
    has_target = true;
  }
  if (has_target) {
    for (int a = 0; a < 2; ++a) {
      const int64_t natural = strides[a] * (in[a] - 1) + opad[a] + (kk[a] - 1) * dil[a] + 1;
      const int64_t total = natural - target[a];
      if (total < 0) return decline("ConvTranspose: output_shape exceeds the un-cropped extent");
      const int64_t half = total / 2;
      pads[a] = ap == "SAME_UPPER" ? half : total - half;
      pads[a + 2] = ap == "SAME_UPPER" ? total - half : half;
    }
  } else if (ap == "VALID") {
    pads.assign(4, 0);
  }
  ohip_convt_desc d{n, c, h, wd, coutg * group, kh, kw, group, strides[0], strides[1], dil[0], dil[1],
                    pads[0], pads[1], pads[2], pads[3], opad[0], opad[1], dt};
  const int64_t oh = ohip_conv_transpose_out_dim(h, strides[0], opad[0], kh, dil[0], pads[0], pads[2]);
  const int64_t ow = ohip_conv_transpose_out_dim(wd, strides[1], opad[1], kw, dil[1], pads[1], pads[3]);
  if (oh < 0 || ow < 0) return decline("ConvTranspose: pads exceed the un-cropped extent");
  ohip_tuning tun;
  ohip_get_tuning(ctx, &tun);
  if (!any_resident(nd) && !ohip_conv_admits(&tun, d.cout, (c / group) * kh * kw, n * h * wd))
    return decline("ConvTranspose: gate");

  std::string name = wkey_name(w), label = "ConvTranspose.W";
  ohip_weight_key key{name.c_str(), label.c_str()};
  const bool cache = w->is_initializer && !name.empty();
  ohip_weight* wt = nullptr;
  int rc = ohip_weight_conv_transpose(ctx, cache ? &key : nullptr, w->dtype, w->data, c, coutg, kh, kw, strides[0],
                                      strides[1], pads[0], pads[1], dil[0], dil[1], group, dt, &wt);
  if (rc) return rc;
  Stage st(ctx);
  const void* xd = st.operand(x);
  const void* bd = nullptr;
  std::vector<char> bconv;
  if (b) {
    if (numel(b) != d.cout) {
      if (!cache) ohip_weight_release(wt);
      return decline("ConvTranspose: bias length");
    }
    bconv.resize((size_t)d.cout * ebytes(dt));
    for (int64_t i = 0; i < d.cout; ++i) put_elem(dt, bconv.data(), i, host_at(b, i));
    bd = st.cached(b, "ConvTranspose.B", dt, bconv.data(), bconv.size());
  }
  const size_t obytes = (size_t)(n * d.cout * oh * ow) * ebytes(dt);
  void* yd = st.alloc(obytes);
  if (!xd || !yd || (b && !bd)) { if (!cache) ohip_weight_release(wt); return OHIP_E_NOMEM; }
  rc = ohip_conv_transpose2d(ctx, &d, xd, wt, bd, yd);
  if (!cache) ohip_weight_release(wt);
  if (rc) return rc;
  set_out(out, dt, {n, d.cout, oh, ow});
  return finish_output(ctx, st, placement, out, yd, obytes, dt);
}

// ------------------------------------------------------------------ Gemm / MatMul
// MatMul whose B is batched (or already on the device): both operands on the
// device, the batch bookkeeping of typed_matmul_batch_info (math_typed.rs:85-115,
// numpy broadcasting of the batch prefixes; slice s reads A slice s % a_batches
// and B slice s % b_batches, math_typed.rs:352-369).
int do_matmul_batched(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor *a = input(nd, 0), *b = input(nd, 1);
  const int dt = a->dtype;
  if (dt != OHIP_F32 && dt != OHIP_F16 && dt != OHIP_BF16) return decline("MatMul: dtype");
  if (b->device && b->dtype != dt) return decline("MatMul: operand dtypes differ");
  if (a->rank < 2 || b->rank < 2) return decline("MatMul: batched operands must be at least 2-D");
  const int64_t m = a->shape[a->rank - 2], k = a->shape[a->rank - 1];
  const int64_t k2 = b->shape[b->rank - 2], n = b->shape[b->rank - 1];
  if (k != k2) return decline("MatMul: K");
  std::vector<int64_t> ab(a->shape, a->shape + a->rank - 2), bb(b->shape, b->shape + b->rank - 2);
  const size_t r = std::max(ab.size(), bb.size());
  std::vector<int64_t> ob(r, 1);
  for (size_t i = 0; i < r; ++i) {
    const int64_t x = i + ab.size() >= r ? ab[i + ab.size() - r] : 1;
    const int64_t y = i + bb.size() >= r ? bb[i + bb.size() - r] : 1;
    if (x != y && x != 1 && y != 1) return decline("MatMul: batch dimensions do not broadcast");
    ob[i] = std::max(x, y);
  }
  int64_t batch = 1, a_batches = 1, b_batches = 1;
  for (auto v : ob) batch *= v;
  for (auto v : ab) a_batches *= v;
  for (auto v : bb) b_batches *= v;
  if (m == 0 || n == 0 || k == 0 || batch == 0) return decline("MatMul: empty");
  ohip_tuning tun;
  ohip_get_tuning(ctx, &tun);
  if (!any_resident(nd) && !ohip_gemm_admits(&tun, m * batch, k, n, false)) return decline("MatMul: gate");
  Stage st(ctx);
  const void* ad = st.operand(a);
  const void* bd = st.operand(b);
  std::vector<int64_t> oshape = ob;
  oshape.push_back(m);
  oshape.push_back(n);
  const size_t obytes = (size_t)(batch * m * n) * ebytes(dt);
  void* yd = st.alloc(obytes);
  if (!ad || !bd || !yd) return OHIP_E_NOMEM;
  ohip_matmul_desc d{m, k, n, batch, a_batches, b_batches, dt};
  int rc = ohip_matmul(ctx, &d, ad, bd, yd);
  if (rc) return rc;
  set_out(out, dt, oshape);
  return finish_output(ctx, st, placement, out, yd, obytes, dt);
}

int do_gemm(ohip_ctx* ctx, const ohip_node* nd, bool is_matmul, int placement, ohip_output* out) {
  const ohip_tensor *a = input(nd, 0), *b = input(nd, 1), *c = is_matmul ? nullptr : input(nd, 2);
  if (!a || !b) return decline("Gemm: missing input");
  if (is_matmul && (b->rank > 2 || b->device)) return do_matmul_batched(ctx, nd, placement, out);
  if (!host_only(b) || (c && !host_only(c))) return decline("Gemm: B / C must be host tensors");
  const int dt = a->dtype;
  if (dt != OHIP_F32 && dt != OHIP_F16 && dt != OHIP_BF16) return decline("Gemm: dtype");
  float alpha = 1.0f, beta = 1.0f;
  int ta = 0, tb = 0;
  int64_t m, k, n;
  std::vector<int64_t> oshape;
  if (is_matmul) {
    // matmul_f32_into (math_typed.rs:334-423) with a shared 2-D (or 1-D) B
    // collapses the batch into M (oxionnx-cuda/src/matmul.rs:189-252).
    if (b->rank == 1) { k = b->shape[0]; n = 1; }
    else if (b->rank == 2) { k = b->shape[0]; n = b->shape[1]; }
    else return decline("MatMul: batched B");
    if (a->rank == 1) { m = 1; if (a->shape[0] != k) return decline("MatMul: K"); }
    else {
      if (a->shape[a->rank - 1] != k) return decline("MatMul: K");
      m = 1;
      for (int i = 0; i < a->rank - 1; ++i) m *= a->shape[i];
    }
    for (int i = 0; i + 1 < a->rank; ++i) oshape.push_back(a->shape[i]);
    if (b->rank == 2) oshape.push_back(n);
  } else {
    // GemmOp (registry/math_ops/matmul_gemm.rs:130-170)
    if (a->rank != 2 || b->rank != 2) return decline("Gemm: rank");
    alpha = attr_f(nd, "alpha", 1.0f);
    beta = attr_f(nd, "beta", 1.0f);
    ta = (int)attr_i(nd, "transA", 0);
    tb = (int)attr_i(nd, "transB", 0);
    m = ta ? a->shape[1] : a->shape[0];
    k = ta ? a->shape[0] : a->shape[1];
    int64_t kb = tb ? b->shape[1] : b->shape[0];
    n = tb ? b->shape[0] : b->shape[1];
    if (k != kb) return decline("Gemm: K");
    oshape = {m, n};
  }
  if (m == 0 || n == 0 || k == 0) return decline("Gemm: empty");
  ohip_tuning tun;
  ohip_get_tuning(ctx, &tun);
  const bool cache = b->is_initializer && b->name && *b->name;
  if (!any_resident(nd) && !ohip_gemm_admits(&tun, m, k, n, cache)) return decline("Gemm: gate");
  std::string name = wkey_name(b), label = std::string(is_matmul ? "MatMul.B" : "Gemm.B");
  ohip_weight_key key{name.c_str(), label.c_str()};
  ohip_weight* wt = nullptr;
  int rc = ohip_weight_gemm(ctx, cache ? &key : nullptr, b->dtype, b->data, k, n, tb, dt, &wt);
  if (rc) return rc;
  Stage st(ctx);
  const void* ad = st.operand(a);
  // C: scalar, [n] / [1,n] row, [m,n] full; any other broadcast is expanded on the host
  int c_kind = OHIP_C_NONE;
  const void* cd = nullptr;
  std::vector<char> cbuf;
  if (c) {
    const int64_t ce = numel(c);
    const int64_t eb = ebytes(dt);
    int64_t cr = 1, cc = 1;
    if (c->rank >= 1) cc = c->shape[c->rank - 1];
    if (c->rank >= 2) cr = c->shape[c->rank - 2];
    if ((cr != 1 && cr != m) || (cc != 1 && cc != n) || ce != cr * cc) { ohip_weight_release(wt); return decline("Gemm: C shape"); }
    if (ce == 1) c_kind = OHIP_C_SCALAR;
    else if (cr == 1 && cc == n) c_kind = OHIP_C_ROW;
    else c_kind = OHIP_C_FULL;
    const int64_t len = c_kind == OHIP_C_SCALAR ? 1 : c_kind == OHIP_C_ROW ? n : m * n;
    cbuf.resize((size_t)(len * eb));
    for (int64_t i = 0; i < len; ++i) {
      int64_t r = c_kind == OHIP_C_FULL ? i / n : 0, col = c_kind == OHIP_C_SCALAR ? 0 : i % n;
      put_elem(dt, cbuf.data(), i, host_at(c, (cr == 1 ? 0 : r) * cc + (cc == 1 ? 0 : col)));
    }
    cd = st.cached(c, is_matmul ? "MatMul.C" : "Gemm.C", dt, cbuf.data(), cbuf.size());
  }
  const size_t obytes = (size_t)(m * n) * ebytes(dt);
  void* yd = st.alloc(obytes);
  if (!ad || !yd || (c && !cd)) { if (!cache) ohip_weight_release(wt); return OHIP_E_NOMEM; }
  ohip_gemm_desc d{m, k, n, dt, ta, alpha, beta, c_kind, OHIP_ACT_NONE, 0.0f, 0.0f, 0, 0};
  rc = ohip_gemm(ctx, &d, ad, wt, cd, yd);
  if (!cache) ohip_weight_release(wt);
  if (rc) return rc;
  set_out(out, dt, oshape);
  return finish_output(ctx, st, placement, out, yd, obytes, dt);
}

// ------------------------------------------------------------------ integer MatMul
int do_qmatmul(ohip_ctx* ctx, const ohip_node* nd, bool qlinear, int placement, ohip_output* out) {
  // QLinearMatMul: a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp
  // MatMulInteger: a, b, a_zp, b_zp
  const ohip_tensor* a = input(nd, 0);
  const ohip_tensor* b = input(nd, qlinear ? 3 : 1);
  const ohip_tensor* azp_t = input(nd, qlinear ? 2 : 2);
  const ohip_tensor* bzp_t = input(nd, qlinear ? 5 : 3);
  if (!a || !b || !host_only(a) || !host_only(b)) return decline("integer MatMul: operands must be host tensors");
  if (b->rank != 2 || a->rank < 1) return decline("integer MatMul: B must be 2-D");
  const int64_t k = b->shape[0], n = b->shape[1];
  if (a->shape[a->rank - 1] != k) return decline("integer MatMul: K");
  int64_t m = 1;
  for (int i = 0; i + 1 < a->rank; ++i) m *= a->shape[i];
  if (m == 0 || n == 0 || k == 0) return decline("integer MatMul: empty");
  std::vector<int32_t> azp, bzp, yzp;
  if (!zp_lanes(azp_t, azp) || !zp_lanes(bzp_t, bzp)) return decline("integer MatMul: zero point");
  if (azp.size() != 1 && (int64_t)azp.size() != m) return decline("integer MatMul: a_zero_point length");
  if (bzp.size() != 1 && (int64_t)bzp.size() != n) return decline("integer MatMul: b_zero_point length");
  float as = 1.0f, bs = 1.0f, ys = 1.0f;
  int32_t lo = 0, hi = 0;
  const ohip_tensor* yzp_t = nullptr;
  if (qlinear) {
    yzp_t = input(nd, 7);
    if (!scale_first(input(nd, 1), &as) || !scale_first(input(nd, 4), &bs) || !scale_first(input(nd, 6), &ys))
      return decline("QLinearMatMul: scale");
    if (!zp_lanes(yzp_t, yzp)) return decline("QLinearMatMul: y_zero_point");
    sat_range(yzp_t, yzp, azp, &lo, &hi);
  }
  ohip_tuning tun;
  ohip_get_tuning(ctx, &tun);
  const bool cache = b->is_initializer && b->name && *b->name;
  if (!any_resident(nd) && !ohip_gemm_admits(&tun, m, k, n, cache)) return decline("integer MatMul: gate");
  std::vector<uint8_t> abytes, bbytes;
  int adt, bdt;
  if (!to_bytes(a, abytes, &adt) || !to_bytes(b, bbytes, &bdt)) return decline("integer MatMul: lanes outside 8 bits");
  std::string name = wkey_name(b), label = std::string(qlinear ? "QLinearMatMul.B" : "MatMulInteger.B");
  ohip_weight_key key{name.c_str(), label.c_str()};
  ohip_weight* wt = nullptr;
  // only b_scale[0] is read, exactly like the reference's scale_input
  int rc = ohip_weight_qgemm(ctx, cache ? &key : nullptr, bdt, bbytes.data(), k, n, 0, bzp.data(), (int)bzp.size(),
                             qlinear ? &bs : nullptr, qlinear ? 1 : 0, &wt);
  if (rc) return rc;
  Stage st(ctx);
  const void* ad = st.operand(a, abytes.data(), abytes.size());
  const size_t obytes = (size_t)(m * n) * 4;
  void* yd = st.alloc(obytes);
  if (!ad || !yd) { if (!cache) ohip_weight_release(wt); return OHIP_E_NOMEM; }
  ohip_qgemm_desc d{m, k, n, adt, azp.data(), (int)azp.size(), qlinear ? OHIP_QOUT_F32 : OHIP_QOUT_I32,
                    as, ys, qlinear ? yzp[0] : 0, lo, hi, 0, 0};
  rc = ohip_qgemm(ctx, &d, ad, wt, yd);
  if (!cache) ohip_weight_release(wt);
  if (rc) return rc;
  std::vector<int64_t> oshape;
  for (int i = 0; i + 1 < a->rank; ++i) oshape.push_back(a->shape[i]);
  oshape.push_back(n);
  set_out(out, qlinear ? OHIP_F32 : OHIP_I32, oshape);
  return finish_output(ctx, st, placement, out, yd, obytes, qlinear ? OHIP_F32 : OHIP_I32);
}

// ------------------------------------------------------------------ integer Conv
// The fused quantised tail DequantizeLinear -> Silu -> QuantizeLinear of a
// QLinearConv output as a byte -> byte table.  Each entry is computed exactly
// as the three reference nodes compute it, in f32 on the host:
//   dequantize_linear_axis  (indexing/quantize.rs:162-190): (q - zp) * scale
//   SiLUOp                  (registry/nn_ops/activations.rs:477-479): x / (1 + exp(-x))
//   quantize_linear_axis    (indexing/quantize.rs:114-150): round_ties_even(x / s) + zp, clamped
// so the table reproduces the unfused chain bit for bit.
bool silu_table(const ohip_node* nd, bool in_signed, int32_t in_zp, float in_scale, uint8_t* table, int* out_dt) {
  if (attr_s(nd, "activation") != "silu") return false;
  const float ys = attr_f(nd, "activation_y_scale", NAN);
  if (!std::isfinite(ys) || ys == 0.0f) return false;
  // saturation_range (quantize.rs:58-66): no zero point -> u8; a zero point
  // above 127 -> u8; any other zero point -> i8
  const bool has_zp = find_attr(nd, "activation_y_zero_point") != nullptr;
  const int64_t yz = attr_i(nd, "activation_y_zero_point", 0);
  const bool u8 = !has_zp || yz > 127;
  const float lo = u8 ? 0.0f : -128.0f, hi = u8 ? 255.0f : 127.0f;
  for (int b = 0; b < 256; ++b) {
    const int32_t q = in_signed ? (int32_t)(int8_t)b : b;
    const float x = ((float)q - (float)in_zp) * in_scale;
    const float s = x / (1.0f + std::exp(-x));
    float v = s / ys;
    float r = std::isfinite(v) ? std::nearbyint(v) : v;
    float o = r + (float)yz;
    o = o < lo ? lo : (o > hi ? hi : o);
    table[b] = (uint8_t)((int32_t)o & 0xff);
  }
  *out_dt = u8 ? OHIP_U8 : OHIP_I8;
  return true;
}

int do_qconv(ohip_ctx* ctx, const ohip_node* nd, bool qlinear, int placement, ohip_output* out) {
  // QLinearConv: x, x_scale, x_zp, w, w_scale, w_zp, y_scale, y_zp, B
  // ConvInteger: x, w, x_zp, w_zp
  const ohip_tensor* x = input(nd, 0);
  const ohip_tensor* w = input(nd, qlinear ? 3 : 1);
  const ohip_tensor* xzp_t = input(nd, 2);
  const ohip_tensor* wzp_t = input(nd, qlinear ? 5 : 3);
  const ohip_tensor* bias = qlinear ? input(nd, 8) : nullptr;
  if (!x || !w || !host_only(w)) return decline("integer Conv: the filter must be a host tensor");
  if (x->device && (x->dtype != OHIP_U8 && x->dtype != OHIP_I8)) return decline("integer Conv: resident X must be bytes");
  const bool x_nhwc = x->device && ohip_dtensor_layout(x->device) == OHIP_NHWC;
  if (x->device && !x_nhwc && ohip_dtensor_layout(x->device) != OHIP_NCHW)
    return decline("integer Conv: resident input layout");
  Geo g;
  std::string why;
  if (!conv_geometry(nd, x, w, &g, &why)) return decline(why);
  const int64_t cg = g.c / g.group;
  std::vector<int32_t> xzp, wzp, yzp;
  if (!zp_lanes(xzp_t, xzp) || !zp_lanes(wzp_t, wzp)) return decline("integer Conv: zero point");
  if (wzp.size() != 1 && (int64_t)wzp.size() != g.cout) return decline("integer Conv: w_zero_point length");
  float xs = 1.0f, ys = 1.0f;
  std::vector<float> ws;
  int32_t lo = 0, hi = 0;
  const ohip_tensor* yzp_t = nullptr;
  if (qlinear) {
    yzp_t = input(nd, 7);
    const ohip_tensor* ws_t = input(nd, 4);
    if (!scale_first(input(nd, 1), &xs) || !scale_first(input(nd, 6), &ys) || !host_only(ws_t) || numel(ws_t) == 0)
      return decline("QLinearConv: scale");
    if (numel(ws_t) != 1 && numel(ws_t) != g.cout) return decline("QLinearConv: w_scale length");
    for (int64_t i = 0; i < numel(ws_t); ++i) {
      double v = host_at(ws_t, i);
      if (!std::isfinite(v)) return decline("QLinearConv: w_scale");
      ws.push_back((float)v);
    }
    if (!zp_lanes(yzp_t, yzp)) return decline("QLinearConv: y_zero_point");
    std::vector<int32_t> x0{xzp[0]};
    sat_range(yzp_t, yzp, x0, &lo, &hi);
  }
  std::vector<int32_t> bias_i;
  if (bias) {
    if (!host_only(bias) || numel(bias) != g.cout) return decline("QLinearConv: bias length");
    for (int64_t i = 0; i < g.cout; ++i) {
      int32_t v;
      if (!lane_int(host_at(bias, i), &v)) return decline("QLinearConv: bias");
      bias_i.push_back(v);
    }
  }
  // Output form: the requantised bytes when the caller keeps the result on
  // the device and the range is one byte type, else the reference's f32 lanes.
  int out_kind = qlinear ? OHIP_QOUT_F32 : OHIP_QOUT_I32;
  int out_dt = qlinear ? OHIP_F32 : OHIP_I32;
  if (qlinear && placement == OHIP_PLACE_DEVICE) {
    if (lo == 0 && hi == 255) { out_kind = OHIP_QOUT_U8; out_dt = OHIP_U8; }
    else if (lo == -128 && hi == 127) { out_kind = OHIP_QOUT_I8; out_dt = OHIP_I8; }
  }
  uint8_t table[256];
  bool fused = false;
  if (!attr_s(nd, "activation").empty()) {
    if (!qlinear || (out_kind != OHIP_QOUT_U8 && out_kind != OHIP_QOUT_I8))
      return decline("integer Conv: a fused tail needs a resident byte output");
    int tdt;
    if (!silu_table(nd, out_kind == OHIP_QOUT_I8, yzp[0], ys, table, &tdt)) return decline("integer Conv: fused tail");
    fused = true;
    out_dt = tdt;
  }
  ohip_tuning tun;
  ohip_get_tuning(ctx, &tun);
  if (!any_resident(nd) && !ohip_conv_admits(&tun, g.cout, cg * g.kh * g.kw, g.n * g.oh * g.ow))
    return decline("integer Conv: gate");
  std::vector<uint8_t> xb, wb;
  int xdt, wdt;
  if (x->device) xdt = x->dtype;
  else if (!to_bytes(x, xb, &xdt)) return decline("integer Conv: lanes outside 8 bits");
  if (!to_bytes(w, wb, &wdt)) return decline("integer Conv: lanes outside 8 bits");
  const bool cache = w->is_initializer && w->name && *w->name;
  std::string name = wkey_name(w), label = std::string(qlinear ? "QLinearConv.W" : "ConvInteger.W");
  ohip_weight_key key{name.c_str(), label.c_str()};
  ohip_weight* wt = nullptr;
  int rc = ohip_weight_qconv(ctx, cache ? &key : nullptr, wdt, wb.data(), g.cout, cg, g.kh, g.kw, wzp.data(),
                             (int)wzp.size(), qlinear ? ws.data() : nullptr, qlinear ? (int)ws.size() : 0, &wt);
  if (rc) return rc;
  Stage st(ctx);
  const void* xd = x->device ? ohip_dtensor_ptr(x->device) : st.operand(x, xb.data(), xb.size());
  const void* bd = bias ? st.cached(bias, "QLinearConv.B", OHIP_I32, bias_i.data(), bias_i.size() * 4) : nullptr;
  const size_t ob = (out_kind == OHIP_QOUT_U8 || out_kind == OHIP_QOUT_I8) ? 1 : 4;
  const size_t obytes = (size_t)(g.n * g.cout * g.oh * g.ow) * ob;
  // A resident byte output stays NHWC (the next convolution's staging
  // layout) when its channels fill whole 16-byte chunks; the dispatcher
  // converts it for consumers that need NCHW.
  const bool y_nhwc = placement == OHIP_PLACE_DEVICE && ob == 1 && g.group == 1 && !g.rank1 && g.cout % 16 == 0 &&
                      nhwc_residency();
  void* yd = st.alloc(obytes);
  if (!xd || !yd || (bias && !bd)) { if (!cache) ohip_weight_release(wt); return OHIP_E_NOMEM; }
  ohip_qconv_desc d{g.n, g.c, g.h, g.w, g.cout, g.kh, g.kw, g.group, g.sh, g.sw, g.dh, g.dw, g.pt, g.pl, g.pb, g.pr,
                    xdt, xzp[0], out_kind, xs, ys, qlinear ? yzp[0] : 0, lo, hi,
                    x_nhwc ? OHIP_NHWC : OHIP_NCHW, y_nhwc ? OHIP_NHWC : OHIP_NCHW, fused ? table : nullptr,
                    x_nhwc ? ohip_dtensor_pitch_internal(x->device) : 0};
  rc = ohip_qconv2d(ctx, &d, xd, wt, static_cast<const int32_t*>(bd), yd);
  if (!cache) ohip_weight_release(wt);
  if (rc) return rc;
  set_out(out, out_dt, conv_out_shape(g));
  rc = finish_output(ctx, st, placement, out, yd, obytes, out_dt);
  if (rc == OHIP_OK && y_nhwc) rc = ohip_dtensor_set_nhwc_internal(out->device, g.cout);
  return rc;
}

// ================================================================== memory-bound nodes
// Counterparts of the reference CUDA provider's elementwise / broadcast /
// norm / pool / resize / pad / slice / concat / alias arms
// (oxionnx-cuda/src/lib.rs:101-119), plus the quantise / dequantise pair of a
// QDQ graph.  Float nodes run in the input's storage type (f32 or f16, f32
// arithmetic); quantised activations stay bytes on the device.

bool is_float_dt(int dt) { return dt == OHIP_F32 || dt == OHIP_F16; }

// The storage type a node computes in: the first resident float input's
// dtype, else f32 (host tensors are f32 lanes).
int node_float_dtype(const ohip_node* nd) {
  for (int i = 0; i < nd->n_inputs; ++i) {
    const ohip_tensor* t = input(nd, i);
    if (t && t->device) return t->dtype;
  }
  for (int i = 0; i < nd->n_inputs; ++i) {
    const ohip_tensor* t = input(nd, i);
    if (t && t->dtype == OHIP_F16) return OHIP_F16;
  }
  return OHIP_F32;
}

// Device pointer of a float operand in storage type dt: the resident buffer
// (which must already be dt), or a converted upload of a host tensor.
const void* float_operand(Stage& st, const ohip_tensor* t, int dt) {
  if (t->device) return t->dtype == dt ? ohip_dtensor_ptr(t->device) : nullptr;
  if (t->dtype == dt) return st.cached(t, "float operand", dt, t->data, (size_t)numel(t) * ebytes(dt));
  const int64_t n = numel(t);
  std::vector<char> buf((size_t)n * ebytes(dt));
  for (int64_t i = 0; i < n; ++i) put_elem(dt, buf.data(), i, host_at(t, i));
  return st.cached(t, "float operand", dt, buf.data(), buf.size());
}

std::vector<int64_t> shape_of(const ohip_tensor* t) { return std::vector<int64_t>(t->shape, t->shape + t->rank); }

// Host int64 lanes of a small shape-like input (pads, starts, axes, ...).
bool host_ints(const ohip_tensor* t, std::vector<int64_t>& out) {
  out.clear();
  if (!t) return true;
  if (!host_only(t)) return false;
  for (int64_t i = 0; i < numel(t); ++i) {
    const double v = host_at(t, i);
    if (!std::isfinite(v)) return false;
    out.push_back((int64_t)v);
  }
  return true;
}

int output_device(ohip_ctx* ctx, Stage& st, int placement, ohip_output* out, int dt, const std::vector<int64_t>& shape,
                  void* yd, size_t bytes) {
  // Host placement returns the reference Tensor's f32 lanes.
  set_out(out, dt, shape);
  if (placement == OHIP_PLACE_DEVICE || dt == OHIP_F32) return finish_output(ctx, st, placement, out, yd, bytes, dt);
  std::vector<uint8_t> raw(bytes);
  int rc = ohip_memcpy_d2h(ctx, raw.data(), yd, bytes);
  if (rc) return rc;
  const int64_t n = bytes / std::max(1, ebytes(dt));
  float* f = static_cast<float*>(std::malloc((size_t)std::max<int64_t>(n, 1) * 4));
  if (!f) return OHIP_E_NOMEM;
  ohip_tensor view{};
  view.dtype = dt;
  view.data = raw.data();
  for (int64_t i = 0; i < n; ++i) f[i] = (float)host_at(&view, i);
  out->dtype = OHIP_F32;
  out->data = f;
  return OHIP_OK;
}

// ---------------------------------------------------------------- unary
int do_unary(ohip_ctx* ctx, const ohip_node* nd, int op, int placement, ohip_output* out) {
  const ohip_tensor* x = input(nd, 0);
  if (!x) return decline("unary: missing input");
  const int dt = node_float_dtype(nd);
  if (!is_float_dt(dt)) return decline("unary: dtype");
  float alpha = 0.0f;
  if (op == ohip::UN_LEAKY_RELU) alpha = attr_f(nd, "alpha", 0.01f);
  Stage st(ctx);
  const void* xd = float_operand(st, x, dt);
  const int64_t n = numel(x);
  const size_t bytes = (size_t)n * ebytes(dt);
  void* yd = st.alloc(bytes);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_unary(dt, xd, yd, n, op, alpha, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  return output_device(ctx, st, placement, out, dt, shape_of(x), yd, bytes);
}

// ---------------------------------------------------------------- binary (numpy broadcasting)
// The broadcast plan of a (rank ra) against b (rank rb): false when the
// shapes do not broadcast or the rank exceeds the kernel's.
bool bcast_plan(const int64_t* as, int ra, const int64_t* bs, int rb, ohip::BcastPlan* p, std::vector<int64_t>* oshape,
                int64_t* n_out) {
  const int rank = std::max(ra, rb);
  if (rank > ohip::kMaxRank) return false;
  *p = ohip::BcastPlan{};
  p->rank = rank;
  int64_t sa = 1, sb = 1, n = 1;
  oshape->assign((size_t)rank, 0);
  for (int d = 0; d < rank; ++d) {
    const int slot = ohip::kMaxRank - 1 - d;
    const int ia = ra - 1 - d, ib = rb - 1 - d;
    const int64_t ea = ia >= 0 ? as[ia] : 1, eb = ib >= 0 ? bs[ib] : 1;
    if (ea != eb && ea != 1 && eb != 1) return false;
    const int64_t e = ea == 1 ? eb : ea;
    p->shape[slot] = e;
    p->sa[slot] = ea == 1 ? 0 : sa;
    p->sb[slot] = eb == 1 ? 0 : sb;
    sa *= ea;
    sb *= eb;
    n *= e;
    (*oshape)[(size_t)(rank - 1 - d)] = e;
  }
  *n_out = n;
  return true;
}

int do_binary(ohip_ctx* ctx, const ohip_node* nd, int op, int placement, ohip_output* out) {
  const ohip_tensor *a = input(nd, 0), *b = input(nd, 1);
  if (!a || !b) return decline("binary: missing input");
  const int dt = node_float_dtype(nd);
  if (!is_float_dt(dt)) return decline("binary: dtype");
  if (std::max(a->rank, b->rank) > ohip::kMaxRank) return decline("binary: rank");
  ohip::BcastPlan p{};
  std::vector<int64_t> oshape;
  int64_t n = 0;
  if (!bcast_plan(a->shape, a->rank, b->shape, b->rank, &p, &oshape, &n))
    return decline("binary: shapes do not broadcast");
  const bool same = numel(a) == n && numel(b) == n;
  Stage st(ctx);
  const void* ad = float_operand(st, a, dt);
  const void* bd = float_operand(st, b, dt);
  const size_t bytes = (size_t)n * ebytes(dt);
  void* yd = st.alloc(bytes);
  if (!ad || !bd || !yd) return ad && bd ? OHIP_E_NOMEM : decline("binary: resident operand dtype");
  hipError_t e = ohip::run_binary(dt, ad, bd, yd, n, p, same, op, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  return output_device(ctx, st, placement, out, dt, oshape, yd, bytes);
}

// ---------------------------------------------------------------- instance normalisation
// OxiInstanceNorm (registry/oxi_instance_norm.rs:135-146): no affine term.
// InstanceNormalization (nn/normalization.rs:251-280): per-channel scale, B.
// This provider's fused AdaIN form of OxiInstanceNorm (the optimizer-side
// fusion of OxiInstanceNorm -> Mul(gamma) -> Add(beta) [-> Relu], the
// modulation of style-based generators): inputs 1 / 2 are resident [N, S]
// style rows; gamma of sample n, channel c is element n * S + scale_offset + c
// of input 1 and beta the same of input 2 at bias_offset; "activation" may be
// "relu".  The arithmetic is the unfused chain's: norm, then * gamma, then
// + beta, then the activation, each in f32.
int do_instnorm(ohip_ctx* ctx, const ohip_node* nd, bool affine, int placement, ohip_output* out) {
  const ohip_tensor* x = input(nd, 0);
  if (!x || x->rank < 3) return decline("InstanceNorm: rank < 3");
  const int dt = node_float_dtype(nd);
  if (!is_float_dt(dt)) return decline("InstanceNorm: dtype");
  const int64_t N = x->shape[0], C = x->shape[1];
  int64_t spatial = 1;
  for (int i = 2; i < x->rank; ++i) spatial *= x->shape[i];
  if (spatial == 0 || N * C == 0) return decline("InstanceNorm: empty");
  const float eps = attr_f(nd, "epsilon", 1e-5f);
  Stage st(ctx);
  ohip::NormAffine aff{nullptr, nullptr, 0, 0, 0, ohip::UN_IDENTITY, 0.0f};
  std::vector<float> sc, bi;
  if (affine) {
    const ohip_tensor *s = input(nd, 1), *b = input(nd, 2);
    if (!s || !b || !host_only(s) || !host_only(b) || numel(s) != C || numel(b) != C)
      return decline("InstanceNormalization: scale / B");
    for (int64_t i = 0; i < C; ++i) { sc.push_back((float)host_at(s, i)); bi.push_back((float)host_at(b, i)); }
    aff.scale = st.cached(s, "InstanceNormalization.scale", OHIP_F32, sc.data(), sc.size() * 4);
    aff.bias = st.cached(b, "InstanceNormalization.B", OHIP_F32, bi.data(), bi.size() * 4);
    if (!aff.scale || !aff.bias) return OHIP_E_NOMEM;
  } else if (nd->n_inputs >= 3 && input(nd, 1) && input(nd, 2)) {
    const ohip_tensor *g = input(nd, 1), *b = input(nd, 2);
    if (!g->device || !b->device || g->dtype != dt || b->dtype != dt || g->rank != 2 || b->rank != 2 ||
        g->shape[0] != N || b->shape[0] != N || g->shape[1] != b->shape[1])
      return decline("OxiInstanceNorm: modulation operands must be resident [N, S] rows of the input's dtype");
    const int64_t so = attr_i(nd, "scale_offset", 0), bo = attr_i(nd, "bias_offset", 0), S = g->shape[1];
    if (so < 0 || bo < 0 || so + C > S || bo + C > S) return decline("OxiInstanceNorm: modulation offsets");
    const int eb = ebytes(dt);
    aff.scale = static_cast<const char*>(ohip_dtensor_ptr(g->device)) + so * eb;
    aff.bias = static_cast<const char*>(ohip_dtensor_ptr(b->device)) + bo * eb;
    aff.per_sample = 1;
    aff.stride = S;
    aff.same_type = 1;
    std::string act = attr_s(nd, "activation");
    if (act == "relu") aff.act = ohip::UN_RELU;
    else if (!act.empty()) return decline("OxiInstanceNorm: activation");
  } else if (nd->n_inputs > 1 && (input(nd, 1) || (nd->n_inputs > 2 && input(nd, 2)))) {
    return decline("OxiInstanceNorm: one input or three");
  }
  const void* xd = float_operand(st, x, dt);
  const size_t bytes = (size_t)numel(x) * ebytes(dt);
  void* yd = st.alloc(bytes);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_instnorm(dt, xd, yd, N * C, spatial, (int)C, eps, aff, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  return output_device(ctx, st, placement, out, dt, shape_of(x), yd, bytes);
}

// ---------------------------------------------------------------- Resize (nearest, rank 4)
// resolve_plan's scales branch (resize.rs:372-420): out = floor(in * scale)
// in f32; only H and W may change.
int do_resize(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor* x = input(nd, 0);
  if (!x || x->rank != 4) return decline("Resize: rank 4 only");
  if (attr_s(nd, "mode") != "nearest") return decline("Resize: nearest only");
  if (find_attr(nd, "axes")) return decline("Resize: axes");
  const ohip_tensor* scales = nd->n_inputs >= 3 ? input(nd, 2) : input(nd, 1);
  if (nd->n_inputs >= 4 && input(nd, 3)) return decline("Resize: sizes");
  if (!scales || !host_only(scales) || numel(scales) != 4) return decline("Resize: scales");
  float s[4];
  for (int i = 0; i < 4; ++i) s[i] = (float)host_at(scales, i);
  if (s[0] != 1.0f || s[1] != 1.0f || !(s[2] > 0.0f) || !(s[3] > 0.0f) || !std::isfinite(s[2]) || !std::isfinite(s[3]))
    return decline("Resize: N / C scales");
  std::string cm = attr_s(nd, "coordinate_transformation_mode"), nm = attr_s(nd, "nearest_mode");
  ohip::ResizePlan p{};
  if (cm.empty() || cm == "half_pixel") p.coord = ohip::RZ_HALF_PIXEL;
  else if (cm == "asymmetric") p.coord = ohip::RZ_ASYMMETRIC;
  else if (cm == "align_corners") p.coord = ohip::RZ_ALIGN_CORNERS;
  else if (cm == "pytorch_half_pixel") p.coord = ohip::RZ_PYTORCH_HALF_PIXEL;
  else if (cm == "tf_half_pixel_for_nn") p.coord = ohip::RZ_TF_HALF_PIXEL_FOR_NN;
  else return decline("Resize: coordinate_transformation_mode");
  if (nm.empty() || nm == "round_prefer_floor") p.rule = ohip::RZ_ROUND_PREFER_FLOOR;
  else if (nm == "round_prefer_ceil") p.rule = ohip::RZ_ROUND_PREFER_CEIL;
  else if (nm == "floor") p.rule = ohip::RZ_FLOOR;
  else if (nm == "ceil") p.rule = ohip::RZ_CEIL;
  else return decline("Resize: nearest_mode");
  p.ih = (int)x->shape[2]; p.iw = (int)x->shape[3];
  p.oh = (int)std::floor((float)x->shape[2] * s[2]);
  p.ow = (int)std::floor((float)x->shape[3] * s[3]);
  p.sh = s[2]; p.sw = s[3];
  if (p.ih <= 0 || p.iw <= 0 || p.oh <= 0 || p.ow <= 0) return decline("Resize: empty");
  const int dt = x->device ? x->dtype : OHIP_F32;
  const int eb = ebytes(dt);
  // a resident NHWC input (passed only under an "out_nhwc" hint, see
  // takes_nhwc) resizes NHWC -> NHWC
  const bool nhwc = x->device && ohip_dtensor_layout(x->device) == OHIP_NHWC;
  Stage st(ctx);
  const void* xd = st.operand(x);
  const int64_t planes = x->shape[0] * x->shape[1];
  const size_t bytes = (size_t)(planes * p.oh * p.ow) * eb;
  void* yd = st.alloc(bytes);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = nhwc ? ohip::run_resize_nearest_nhwc(eb, xd, yd, x->shape[0], x->shape[1], p,
                                                      (hipStream_t)ohip_ctx_stream(ctx))
                      : ohip::run_resize_nearest(eb, xd, yd, planes, p, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  int rc = output_device(ctx, st, placement, out, dt, {x->shape[0], x->shape[1], p.oh, p.ow}, yd, bytes);
  if (rc == OHIP_OK && nhwc && out->device) rc = ohip_dtensor_set_nhwc_internal(out->device, x->shape[1]);
  return rc;
}

// ---------------------------------------------------------------- Pad
int do_pad(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor* x = input(nd, 0);
  if (!x || x->rank < 1 || x->rank > ohip::kMaxRank) return decline("Pad: rank");
  std::vector<int64_t> pads;
  if (nd->n_inputs >= 2 && input(nd, 1)) {
    if (!host_ints(input(nd, 1), pads)) return decline("Pad: pads must be a host tensor");
  } else {
    pads = attr_ints(nd, "pads");
  }
  if (nd->n_inputs >= 4 && input(nd, 3)) return decline("Pad: axes");
  if ((int)pads.size() != 2 * x->rank) return decline("Pad: pads length");
  for (auto v : pads) if (v < 0) return decline("Pad: negative pads");
  std::string mode = attr_s(nd, "mode");
  ohip::PadPlan p{};
  p.rank = x->rank;
  if (mode.empty() || mode == "constant") p.mode = ohip::PAD_CONSTANT;
  else if (mode == "reflect") p.mode = ohip::PAD_REFLECT;
  else if (mode == "edge") p.mode = ohip::PAD_EDGE;
  else if (mode == "wrap") p.mode = ohip::PAD_WRAP;
  else return decline("Pad: mode");
  const int dt = x->device ? x->dtype : OHIP_F32;
  const int eb = ebytes(dt);
  double value = 0.0;
  if (nd->n_inputs >= 3 && input(nd, 2)) {
    const ohip_tensor* cv = input(nd, 2);
    if (!host_only(cv) || numel(cv) < 1) return decline("Pad: constant_value");
    value = host_at(cv, 0);
  } else if (find_attr(nd, "value")) {
    value = attr_f(nd, "value", 0.0f);
  }
  {
    uint32_t bits = 0;
    if (dt == OHIP_U8 || dt == OHIP_I8) bits = (uint32_t)((int32_t)std::nearbyint(value) & 0xff);
    else { char tmp[4] = {0}; put_elem(dt, tmp, 0, value); std::memcpy(&bits, tmp, (size_t)eb); }
    p.value_bits = bits;
  }
  std::vector<int64_t> oshape((size_t)x->rank);
  int64_t n = 1;
  for (int d = 0; d < x->rank; ++d) {
    p.in[d] = x->shape[d];
    p.begin[d] = pads[(size_t)d];
    p.out[d] = x->shape[d] + pads[(size_t)d] + pads[(size_t)(d + x->rank)];
    if (p.mode != ohip::PAD_CONSTANT && p.in[d] == 0 && p.out[d] > 0) return decline("Pad: empty axis");
    if (p.mode == ohip::PAD_REFLECT && (pads[(size_t)d] >= p.in[d] || pads[(size_t)(d + x->rank)] >= p.in[d]) &&
        p.in[d] > 1)
      return decline("Pad: reflect pad wider than the axis");
    oshape[(size_t)d] = p.out[d];
    n *= p.out[d];
  }
  Stage st(ctx);
  const void* xd = st.operand(x);
  const size_t bytes = (size_t)n * eb;
  void* yd = st.alloc(bytes);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_pad(eb, xd, yd, n, p, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  return output_device(ctx, st, placement, out, dt, oshape, yd, bytes);
}

// ---------------------------------------------------------------- MaxPool (2-D)
// PoolGeometry::resolve + pool_out_dim (conv/pooling.rs:44-90,
// conv/spatial.rs:272-322); dilations, ceil_mode and auto_pad honoured.
int do_maxpool(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor* x = input(nd, 0);
  if (!x || x->rank != 4) return decline("MaxPool: 2-D only");
  if (attr_i(nd, "storage_order", 0) != 0) return decline("MaxPool: storage_order");
  auto ks = attr_ints(nd, "kernel_shape"), strides = attr_ints(nd, "strides"), pads = attr_ints(nd, "pads"),
       dil = attr_ints(nd, "dilations");
  if (ks.size() != 2) return decline("MaxPool: kernel_shape");
  if (strides.empty()) strides = {1, 1};
  if (dil.empty()) dil = {1, 1};
  if (pads.empty()) pads = {0, 0, 0, 0};
  if (strides.size() != 2 || dil.size() != 2 || pads.size() != 4) return decline("MaxPool: attribute rank");
  for (auto v : ks) if (v <= 0) return decline("MaxPool: kernel");
  for (auto v : strides) if (v <= 0) return decline("MaxPool: stride");
  for (auto v : dil) if (v <= 0) return decline("MaxPool: dilation");
  for (auto v : pads) if (v < 0) return decline("MaxPool: pads");
  const bool ceil_mode = attr_i(nd, "ceil_mode", 0) != 0;
  const int64_t ih = x->shape[2], iw = x->shape[3];
  std::string ap = attr_s(nd, "auto_pad");
  if (ap == "VALID") pads = {0, 0, 0, 0};
  else if (ap == "SAME_UPPER" || ap == "SAME_LOWER") {
    for (int a = 0; a < 2; ++a) {
      const int64_t in = a ? iw : ih;
      const int64_t o = (in + strides[(size_t)a] - 1) / strides[(size_t)a];
      const int64_t eff = (ks[(size_t)a] - 1) * dil[(size_t)a] + 1;
      const int64_t need = std::max<int64_t>(0, (o - 1) * strides[(size_t)a] + eff - in), half = need / 2;
      pads[(size_t)a] = ap == "SAME_LOWER" ? need - half : half;
      pads[(size_t)(a + 2)] = need - pads[(size_t)a];
    }
  } else if (!(ap.empty() || ap == "NOTSET")) {
    return decline("MaxPool: auto_pad");
  }
  auto out_dim = [&](int64_t in, int64_t pb, int64_t pe, int64_t k, int64_t d, int64_t s) -> int64_t {
    const int64_t eff = (k - 1) * d + 1, padded = in + pb + pe;
    if (padded < eff) return -1;
    const int64_t span = padded - eff;
    int64_t o = ceil_mode ? (span + s - 1) / s + 1 : span / s + 1;
    if (ceil_mode && o > 1 && (o - 1) * s >= in + pb) o -= 1;
    return o;
  };
  const int64_t oh = out_dim(ih, pads[0], pads[2], ks[0], dil[0], strides[0]);
  const int64_t ow = out_dim(iw, pads[1], pads[3], ks[1], dil[1], strides[1]);
  if (oh <= 0 || ow <= 0) return decline("MaxPool: output extent");
  const int dt = x->device ? x->dtype : OHIP_F32;
  ohip::PoolPlan p{(int)ih, (int)iw, (int)oh, (int)ow, (int)ks[0], (int)ks[1], (int)strides[0], (int)strides[1],
                   (int)pads[0], (int)pads[1], (int)dil[0], (int)dil[1]};
  // a resident NHWC input is pooled in place; the output is compact NHWC
  const bool nhwc = x->device && ohip_dtensor_layout(x->device) == OHIP_NHWC;
  if (nhwc) {
    p.nhwc_c = (int)x->shape[1];
    p.pitch = ohip_dtensor_pitch_internal(x->device);
  }
  Stage st(ctx);
  const void* xd = st.operand(x);
  const int64_t planes = x->shape[0] * x->shape[1];
  const size_t bytes = (size_t)(planes * oh * ow) * ebytes(dt);
  void* yd = st.alloc(bytes);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_maxpool(dt, xd, yd, planes, p, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return e == hipErrorInvalidValue ? decline("MaxPool: dtype") : ohip_hip_error_internal(e, "MaxPool launch");
  int rc = output_device(ctx, st, placement, out, dt, {x->shape[0], x->shape[1], oh, ow}, yd, bytes);
  if (rc == OHIP_OK && nhwc && out->device) rc = ohip_dtensor_set_nhwc_internal(out->device, x->shape[1]);
  return rc;
}

// ---------------------------------------------------------------- Concat (device copy kernels)
int do_concat(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  if (nd->n_inputs < 1) return decline("Concat: no inputs");
  const ohip_tensor* t0 = input(nd, 0);
  if (!t0) return decline("Concat: missing input");
  const int rank = t0->rank;
  int64_t axis = attr_i(nd, "axis", 0);
  if (axis < 0) axis += rank;
  if (axis < 0 || axis >= rank) return decline("Concat: axis");
  int dt = -1;
  for (int i = 0; i < nd->n_inputs; ++i) {
    const ohip_tensor* t = input(nd, i);
    if (t && t->device) { dt = t->dtype; break; }
  }
  if (dt < 0) dt = OHIP_F32;
  const int eb = ebytes(dt);
  std::vector<int64_t> oshape = shape_of(t0);
  oshape[(size_t)axis] = 0;
  int64_t outer = 1, inner = 1;
  for (int d = 0; d < axis; ++d) outer *= t0->shape[d];
  for (int d = axis + 1; d < rank; ++d) inner *= t0->shape[d];
  for (int i = 0; i < nd->n_inputs; ++i) {
    const ohip_tensor* t = input(nd, i);
    if (!t || t->rank != rank) return decline("Concat: rank");
    for (int d = 0; d < rank; ++d)
      if (d != axis && t->shape[d] != t0->shape[d]) return decline("Concat: shapes");
    if (t->device && t->dtype != dt) return decline("Concat: mixed dtypes");
    if (!t->device && dt != OHIP_F32) return decline("Concat: host operand beside byte tensors");
    oshape[(size_t)axis] += t->shape[axis];
  }
  // every input resident NHWC, channel axis (the dispatcher converts any
  // other mix first): rows are pixels, each input adds its channels with its
  // own pixel pitch, the output is compact NHWC
  bool nhwc = rank == 4 && axis == 1;
  for (int i = 0; i < nd->n_inputs && nhwc; ++i) {
    const ohip_tensor* t = input(nd, i);
    nhwc = t->device && ohip_dtensor_layout(t->device) == OHIP_NHWC;
  }
  if (nhwc) {
    outer = t0->shape[0] * t0->shape[2] * t0->shape[3];
    inner = 1;
  }
  Stage st(ctx);
  const size_t row = (size_t)(oshape[(size_t)axis] * inner * eb);
  const size_t bytes = (size_t)outer * row;
  void* yd = st.alloc(bytes);
  if (!yd) return OHIP_E_NOMEM;
  hipStream_t s = (hipStream_t)ohip_ctx_stream(ctx);
  // the inputs in groups of up to kConcatMax, one launch per group
  size_t off = 0;
  ohip::ConcatPlan p{};
  size_t group_off = 0;
  auto flush = [&]() -> int {
    if (p.n == 0) return OHIP_OK;
    p.dst = static_cast<char*>(yd) + group_off;
    const int64_t gw = (int64_t)(off - group_off);
    // rows of the group's part: pitch `row` in the output; a one-group concat
    // writes whole output rows
    if (gw == (int64_t)row) {
      if (ohip::run_concat_rows(p, gw, outer, s) != hipSuccess)
        return ohip_hip_error_internal(hipGetLastError(), "Concat copy");
    } else {
      for (int k = 0; k < p.n; ++k)
        if (p.w[k] && outer &&
            ohip::run_copy2d(p.src[k], p.sp[k], static_cast<char*>(p.dst) + p.off[k], (int64_t)row, p.w[k], outer, s) !=
                hipSuccess)
          return ohip_hip_error_internal(hipGetLastError(), "Concat copy");
    }
    p.n = 0;
    group_off = off;
    return OHIP_OK;
  };
  for (int i = 0; i < nd->n_inputs; ++i) {
    const ohip_tensor* t = input(nd, i);
    const void* td = st.operand(t);
    if (!td) return OHIP_E_NOMEM;
    const size_t w = (size_t)(t->shape[axis] * inner * eb);
    if (p.n == ohip::kConcatMax) {
      int rc = flush();
      if (rc) return rc;
    }
    p.src[p.n] = td;
    p.w[p.n] = (int64_t)w;
    p.sp[p.n] = nhwc ? ohip_dtensor_pitch_internal(t->device) * eb : (int64_t)w;
    p.off[p.n] = (int64_t)(off - group_off);
    ++p.n;
    off += w;
  }
  {
    int rc = flush();
    if (rc) return rc;
  }
  int rc = output_device(ctx, st, placement, out, dt, oshape, yd, bytes);
  if (rc == OHIP_OK && nhwc && out->device) rc = ohip_dtensor_set_nhwc_internal(out->device, oshape[1]);
  return rc;
}

// ---------------------------------------------------------------- Slice (positive steps)
int do_slice(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor* x = input(nd, 0);
  if (!x || x->rank < 1 || x->rank > ohip::kMaxRank) return decline("Slice: rank");
  std::vector<int64_t> starts, ends, axes, steps;
  if (nd->n_inputs >= 3) {
    if (!host_ints(input(nd, 1), starts) || !host_ints(input(nd, 2), ends) ||
        !host_ints(nd->n_inputs >= 4 ? input(nd, 3) : nullptr, axes) ||
        !host_ints(nd->n_inputs >= 5 ? input(nd, 4) : nullptr, steps))
      return decline("Slice: parameters must be host tensors");
  } else {
    starts = attr_ints(nd, "starts");
    ends = attr_ints(nd, "ends");
    axes = attr_ints(nd, "axes");
  }
  if (starts.size() != ends.size()) return decline("Slice: starts / ends");
  if (axes.empty()) for (size_t i = 0; i < starts.size(); ++i) axes.push_back((int64_t)i);
  if (steps.empty()) steps.assign(starts.size(), 1);
  if (axes.size() != starts.size() || steps.size() != starts.size()) return decline("Slice: lengths");
  ohip::SlicePlan p{};
  p.rank = x->rank;
  int64_t stride = 1;
  for (int d = x->rank - 1; d >= 0; --d) {
    p.in_stride[d] = stride;
    stride *= x->shape[d];
    p.start[d] = 0;
    p.step[d] = 1;
    p.out[d] = x->shape[d];
  }
  for (size_t i = 0; i < starts.size(); ++i) {
    int64_t a = axes[i] < 0 ? axes[i] + x->rank : axes[i];
    if (a < 0 || a >= x->rank) return decline("Slice: axis");
    if (steps[i] <= 0) return decline("Slice: non-positive step");
    const int64_t dim = x->shape[a];
    int64_t s = starts[i], e = ends[i];
    if (s < 0) s += dim;
    if (e < 0) e += dim;
    s = std::min(std::max<int64_t>(s, 0), dim);
    e = std::min(std::max<int64_t>(e, 0), dim);
    p.start[a] = s;
    p.step[a] = steps[i];
    p.out[a] = e > s ? (e - s + steps[i] - 1) / steps[i] : 0;
  }
  std::vector<int64_t> oshape(p.out, p.out + x->rank);
  int64_t n = 1;
  for (auto v : oshape) n *= v;
  const int dt = x->device ? x->dtype : OHIP_F32;
  const int eb = ebytes(dt);
  // A resident NHWC input: a whole-chunk channel range (unit step, every
  // other axis whole) is a view with the input's pixel pitch; anything else
  // reads the input's NCHW form.
  Stage st(ctx);
  const void* xnchw = nullptr;
  if (x->device && ohip_dtensor_layout(x->device) == OHIP_NHWC) {
    bool chan_only = x->rank == 4 && (p.step[1] == 1 || p.out[1] <= 1);
    for (int d = 0; d < x->rank && chan_only; ++d)
      if (d != 1 && p.out[d] != x->shape[d]) chan_only = false;
    if (chan_only && placement == OHIP_PLACE_DEVICE && (p.start[1] * eb) % 16 == 0 && (p.out[1] * eb) % 16 == 0 &&
        p.out[1] > 0) {
      ohip_dtensor* t = nullptr;
      int rc = ohip_dtensor_view_nhwc_internal(x->device, p.start[1], p.out[1], &t);
      if (rc) return rc;
      set_out(out, dt, oshape);
      out->device = t;
      return OHIP_OK;
    }
    void* c = st.alloc((size_t)std::max<int64_t>(numel(x) * eb, 16));
    if (!c) return OHIP_E_NOMEM;
    int rc = ohip_dtensor_to_nchw_internal(ctx, x->device, c);
    if (rc) return rc;
    xnchw = c;
  }
  // A resident input whose slice is one contiguous run (every axis before the
  // first sliced one has extent 1 in the output, the axes after it are whole,
  // unit step) becomes a view of the input's buffer: no copy, no launch.  The
  // view starts on a 16-byte boundary, as every freshly allocated tensor does.
  if (!xnchw && x->device && placement == OHIP_PLACE_DEVICE && ohip_dtensor_layout(x->device) == OHIP_NCHW && n > 0) {
    int k = 0;
    while (k < x->rank && p.out[k] == x->shape[k]) ++k;   // first sliced axis
    bool contiguous = true;
    int64_t off = 0;
    for (int d = 0; d < x->rank; ++d) {
      if (d < k) { if (p.out[d] != 1 && x->shape[d] != 1) contiguous = false; }
      else if (d == k) { if (p.step[d] != 1 && p.out[d] > 1) contiguous = false; }
      else if (p.out[d] != x->shape[d]) contiguous = false;
      off += p.start[d] * p.in_stride[d];
    }
    // axes before k are whole; a whole axis of extent > 1 before k breaks it
    for (int d = 0; d < k; ++d) if (x->shape[d] != 1) contiguous = false;
    if (contiguous && (off * eb) % 16 == 0) {
      ohip_dtensor* t = nullptr;
      int rc = ohip_dtensor_view_internal(x->device, x->rank, oshape.data(), (size_t)(off * eb), &t);
      if (rc) return rc;
      set_out(out, dt, oshape);
      out->device = t;
      return OHIP_OK;
    }
  }
  const void* xd = xnchw ? xnchw : st.operand(x);
  const size_t bytes = (size_t)n * eb;
  void* yd = st.alloc(bytes);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_slice(eb, xd, yd, n, p, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  return output_device(ctx, st, placement, out, dt, oshape, yd, bytes);
}

// ---------------------------------------------------------------- shape aliases
// Reshape / Flatten / Squeeze / Unsqueeze of a resident tensor: the output
// shares the input's buffer (oxionnx-cuda's CudaDeviceTensor::alias); a host
// input is declined (the CPU op is a free relabel).
int do_alias(ohip_ctx* ctx, const ohip_node* nd, const std::string& op, int placement, ohip_output* out) {
  const ohip_tensor* x = input(nd, 0);
  if (!x || !x->device || placement != OHIP_PLACE_DEVICE) return decline(op + ": host operand");
  std::vector<int64_t> in = shape_of(x), o;
  int64_t total = 1;
  for (auto v : in) total *= v;
  if (op == "Reshape") {
    std::vector<int64_t> sh;
    if (!host_ints(input(nd, 1), sh)) return decline("Reshape: shape must be a host tensor");
    const bool allowzero = attr_i(nd, "allowzero", 0) != 0;
    int64_t known = 1;
    int infer = -1;
    for (size_t i = 0; i < sh.size(); ++i) {
      int64_t v = sh[i];
      if (v == 0 && !allowzero) { if (i >= in.size()) return decline("Reshape: 0 past rank"); v = in[i]; }
      if (v == -1) { if (infer >= 0) return decline("Reshape: two -1"); infer = (int)i; o.push_back(1); continue; }
      if (v < 0) return decline("Reshape: negative extent");
      o.push_back(v);
      known *= v;
    }
    if (infer >= 0) { if (known == 0 || total % known) return decline("Reshape: -1"); o[(size_t)infer] = total / known; }
  } else if (op == "Flatten") {
    int64_t axis = attr_i(nd, "axis", 1);
    if (axis < 0) axis += (int64_t)in.size();
    if (axis < 0 || axis > (int64_t)in.size()) return decline("Flatten: axis");
    int64_t a = 1;
    for (int64_t i = 0; i < axis; ++i) a *= in[(size_t)i];
    o = {a, a ? total / a : 0};
  } else {
    std::vector<int64_t> axes;
    if (nd->n_inputs >= 2 && input(nd, 1)) {
      if (!host_ints(input(nd, 1), axes)) return decline(op + ": axes must be a host tensor");
    } else {
      axes = attr_ints(nd, "axes");
    }
    if (op == "Squeeze") {
      const int r = (int)in.size();
      std::vector<bool> drop((size_t)r, false);
      if (axes.empty()) for (int i = 0; i < r; ++i) drop[(size_t)i] = in[(size_t)i] == 1;
      for (auto a : axes) {
        if (a < 0) a += r;
        if (a < 0 || a >= r || in[(size_t)a] != 1) return decline("Squeeze: axis");
        drop[(size_t)a] = true;
      }
      for (int i = 0; i < r; ++i) if (!drop[(size_t)i]) o.push_back(in[(size_t)i]);
    } else {
      const int r = (int)(in.size() + axes.size());
      std::vector<bool> ins((size_t)r, false);
      for (auto a : axes) {
        if (a < 0) a += r;
        if (a < 0 || a >= r || ins[(size_t)a]) return decline("Unsqueeze: axis");
        ins[(size_t)a] = true;
      }
      size_t k = 0;
      for (int i = 0; i < r; ++i) o.push_back(ins[(size_t)i] ? 1 : in[k++]);
    }
  }
  int64_t check = 1;
  for (auto v : o) check *= v;
  if (check != total || o.size() > 8) return decline(op + ": element count");
  ohip_dtensor* t = nullptr;
  int rc = ohip_dtensor_alias_internal(x->device, (int)o.size(), o.data(), &t);
  if (rc) return rc;
  set_out(out, x->dtype, o);
  out->device = t;
  return OHIP_OK;
}

// ---------------------------------------------------------------- QuantizeLinear / DequantizeLinear
// Per-tensor parameters only (quantize.rs:96-190).
int do_quantize(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor *x = input(nd, 0), *s = input(nd, 1), *z = input(nd, 2);
  if (!x) return decline("QuantizeLinear: missing input");
  if (x->device && x->dtype != OHIP_F32) return decline("QuantizeLinear: resident input must be f32");
  float scale;
  if (!s || !host_only(s) || numel(s) != 1) return decline("QuantizeLinear: per-tensor scale only");
  scale = (float)host_at(s, 0);
  float zp = 0.0f;
  if (z && numel(z) > 1) return decline("QuantizeLinear: per-tensor zero point only");
  if (z && !host_only(z)) return decline("QuantizeLinear: zero point");
  if (z && numel(z) == 0) return decline("QuantizeLinear: empty zero point");
  if (z) zp = (float)host_at(z, 0);
  // saturation_range (quantize.rs:58-66): the output type follows the zero
  // point's value, as in the reference (its Tensor carries no dtype tag)
  const bool u8 = !z || zp > 127.0f;
  const float lo = u8 ? 0.0f : -128.0f, hi = u8 ? 255.0f : 127.0f;
  Stage st(ctx);
  const void* xd = float_operand(st, x, OHIP_F32);
  const int64_t n = numel(x);
  void* yd = st.alloc((size_t)n);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_quantize(static_cast<const float*>(xd), static_cast<uint8_t*>(yd), n, scale, zp, lo, hi,
                                    (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  return output_device(ctx, st, placement, out, u8 ? OHIP_U8 : OHIP_I8, shape_of(x), yd, (size_t)n);
}

int do_dequantize(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  const ohip_tensor *x = input(nd, 0), *s = input(nd, 1), *z = input(nd, 2);
  if (!x) return decline("DequantizeLinear: missing input");
  if (!s || !host_only(s) || numel(s) != 1) return decline("DequantizeLinear: per-tensor scale only");
  if (z && (!host_only(z) || numel(z) != 1)) return decline("DequantizeLinear: per-tensor zero point only");
  const float scale = (float)host_at(s, 0), zp = z ? (float)host_at(z, 0) : 0.0f;
  Stage st(ctx);
  const void* xd;
  int xdt;
  std::vector<uint8_t> xb;
  if (x->device) {
    xdt = x->dtype;
    if (xdt != OHIP_U8 && xdt != OHIP_I8) return decline("DequantizeLinear: resident input must be bytes");
    xd = ohip_dtensor_ptr(x->device);
  } else {
    if (!to_bytes(x, xb, &xdt)) return decline("DequantizeLinear: lanes outside 8 bits");
    xd = st.operand(x, xb.data(), xb.size());
  }
  const int64_t n = numel(x);
  void* yd = st.alloc((size_t)n * 4);
  if (!xd || !yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_dequantize(static_cast<const uint8_t*>(xd), xdt == OHIP_I8, static_cast<float*>(yd), n,
                                      scale, zp, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  return output_device(ctx, st, placement, out, OHIP_F32, shape_of(x), yd, (size_t)n * 4);
}

// ---------------------------------------------------------------- QLinearAdd
// This provider's fusion of DequantizeLinear(A), DequantizeLinear(B), Add and
// QuantizeLinear (the dequantised residual sum of quantised networks), with
// the ONNX contrib operator's inputs: A, A_scale, A_zero_point, B, B_scale,
// B_zero_point, C_scale, C_zero_point (per-tensor).  Each step is computed as
// the unfused node computes it (do_dequantize, do_binary, do_quantize); the
// output type follows C's zero point as QuantizeLinear's does.
int do_qadd(ohip_ctx* ctx, const ohip_node* nd, int placement, ohip_output* out) {
  if (nd->n_inputs < 7) return decline("QLinearAdd: inputs");
  const ohip_tensor* a = input(nd, 0);
  const ohip_tensor* b = input(nd, 3);
  if (!a || !b) return decline("QLinearAdd: missing operand");
  auto scalar = [&](int i, bool need, float* v) {
    const ohip_tensor* t = input(nd, i);
    if (!t) { *v = 0.0f; return !need; }
    if (!host_only(t) || numel(t) != 1) return false;
    *v = (float)host_at(t, 0);
    return true;
  };
  ohip::QAddArgs q{};
  if (!scalar(1, true, &q.sa) || !scalar(2, false, &q.za) || !scalar(4, true, &q.sb) || !scalar(5, false, &q.zb) ||
      !scalar(6, true, &q.sc) || !scalar(7, false, &q.zc))
    return decline("QLinearAdd: per-tensor scales and zero points only");
  const bool has_zc = input(nd, 7) != nullptr;
  const bool u8 = !has_zc || q.zc > 127.0f;
  q.lo = u8 ? 0.0f : -128.0f;
  q.hi = u8 ? 255.0f : 127.0f;
  const int rank = std::max(a->rank, b->rank);
  if (rank > ohip::kMaxRank) return decline("QLinearAdd: rank");
  ohip::BcastPlan p{};
  p.rank = rank;
  int64_t sa = 1, sb = 1, n = 1;
  std::vector<int64_t> oshape((size_t)rank);
  for (int d = 0; d < rank; ++d) {
    const int slot = ohip::kMaxRank - 1 - d;
    const int ia = a->rank - 1 - d, ib = b->rank - 1 - d;
    const int64_t ea = ia >= 0 ? a->shape[ia] : 1, eb = ib >= 0 ? b->shape[ib] : 1;
    if (ea != eb && ea != 1 && eb != 1) return decline("QLinearAdd: shapes do not broadcast");
    const int64_t e = ea == 1 ? eb : ea;
    p.shape[slot] = e;
    p.sa[slot] = ea == 1 ? 0 : sa;
    p.sb[slot] = eb == 1 ? 0 : sb;
    sa *= ea;
    sb *= eb;
    n *= e;
    oshape[(size_t)(rank - 1 - d)] = e;
  }
  bool same = numel(a) == n && numel(b) == n;
  // both operands resident NHWC of one shape (the dispatcher converts any
  // other NHWC operand first): pixels x channels with each operand's pitch,
  // the output compact NHWC
  const bool nhwc = a->device && b->device && ohip_dtensor_layout(a->device) == OHIP_NHWC &&
                    ohip_dtensor_layout(b->device) == OHIP_NHWC;
  if (nhwc) {
    p = ohip::BcastPlan{};
    p.rank = 2;
    p.shape[ohip::kMaxRank - 2] = a->shape[0] * a->shape[2] * a->shape[3];
    p.shape[ohip::kMaxRank - 1] = a->shape[1];
    p.sa[ohip::kMaxRank - 2] = ohip_dtensor_pitch_internal(a->device);
    p.sb[ohip::kMaxRank - 2] = ohip_dtensor_pitch_internal(b->device);
    p.sa[ohip::kMaxRank - 1] = p.sb[ohip::kMaxRank - 1] = 1;
    same = p.sa[ohip::kMaxRank - 2] == a->shape[1] && p.sb[ohip::kMaxRank - 2] == a->shape[1];
  }
  Stage st(ctx);
  std::vector<uint8_t> ab, bb;
  auto bytes_of = [&](const ohip_tensor* t, std::vector<uint8_t>& hb, int* dt) -> const void* {
    if (t->device) {
      *dt = t->dtype;
      if (*dt != OHIP_U8 && *dt != OHIP_I8) return nullptr;
      return ohip_dtensor_ptr(t->device);
    }
    if (!to_bytes(t, hb, dt)) return nullptr;
    return st.operand(t, hb.data(), hb.size());
  };
  int adt = -1, bdt = -1;
  const void* ad = bytes_of(a, ab, &adt);
  const void* bd = bytes_of(b, bb, &bdt);
  if (!ad || !bd) return decline("QLinearAdd: operands must be 8-bit");
  q.a_signed = adt == OHIP_I8;
  q.b_signed = bdt == OHIP_I8;
  void* yd = st.alloc((size_t)n);
  if (!yd) return OHIP_E_NOMEM;
  hipError_t e = ohip::run_qadd(static_cast<const uint8_t*>(ad), static_cast<const uint8_t*>(bd),
                                static_cast<uint8_t*>(yd), n, p, same, q, (hipStream_t)ohip_ctx_stream(ctx));
  if (e != hipSuccess) return ohip_hip_error_internal(e, "node kernel launch");
  int rc = output_device(ctx, st, placement, out, u8 ? OHIP_U8 : OHIP_I8, oshape, yd, (size_t)n);
  if (rc == OHIP_OK && nhwc && out->device) rc = ohip_dtensor_set_nhwc_internal(out->device, a->shape[1]);
  return rc;
}

}  // namespace

// ------------------------------------------------------------------ public
// is_supported_op (oxionnx-cuda/src/lib.rs:217-275), restricted to this
// provider's dense-contraction arms.
extern "C" int ohip_is_supported_op(const char* op) {
  if (!op) return 0;
  static const char* kOps[] = {"Conv", "ConvTranspose", "Gemm", "MatMul", "QLinearMatMul", "MatMulInteger", "QLinearConv",
                               "ConvInteger", "Relu", "LeakyRelu", "Tanh", "Sigmoid", "Silu", "Identity",
                               "Add", "Sub", "Mul", "Div", "OxiInstanceNorm", "InstanceNormalization", "Resize",
                               "Pad", "MaxPool", "Concat", "Slice", "Reshape", "Flatten", "Squeeze", "Unsqueeze",
                               "QuantizeLinear", "DequantizeLinear", "QLinearAdd", "OhipConvInstanceNorm"};
  for (const char* o : kOps)
    if (std::strcmp(op, o) == 0) return 1;
  return 0;
}

// accepts_resident_slot (oxionnx-cuda/src/lib.rs:419-480): the activation
// slots may be bound from resident tensors; filters, Gemm B / C, quantisation
// parameters and shape-like inputs are read on the host.
extern "C" int ohip_accepts_resident_slot(const char* op, int index) {
  if (!op) return 0;
  static const char* kSlot0[] = {"Conv", "ConvTranspose", "Gemm", "MatMul", "QLinearConv", "Relu", "LeakyRelu", "Tanh", "Sigmoid",
                                 "Silu", "Identity", "InstanceNormalization", "Resize", "Pad",
                                 "MaxPool", "Slice", "Reshape", "Flatten", "Squeeze", "Unsqueeze",
                                 "QuantizeLinear", "DequantizeLinear"};
  for (const char* o : kSlot0)
    if (std::strcmp(op, o) == 0) return index == 0;
  if (!std::strcmp(op, "Add") || !std::strcmp(op, "Sub") || !std::strcmp(op, "Mul") || !std::strcmp(op, "Div"))
    return index == 0 || index == 1;
  if (!std::strcmp(op, "OxiInstanceNorm")) return index >= 0 && index <= 2;
  if (!std::strcmp(op, "OhipConvInstanceNorm")) return index == 0 || index == 3 || index == 4 || index == 5;
  if (!std::strcmp(op, "Concat")) return index >= 0;
  if (!std::strcmp(op, "QLinearAdd")) return index == 0 || index == 3;
  return 0;
}

namespace {

int dispatch_node(ohip_ctx* ctx, const ohip_node* node, int placement, ohip_output* out);

// Whether a node reads resident NHWC operand i in place (device placement
// only): QLinearConv's X (group 1), QLinearAdd's operands when both are NHWC
// of one shape, Concat along channels when every input is NHWC, MaxPool, and
// Slice (a channel range is a view; anything else converts inside do_slice).
bool takes_nhwc(ohip_ctx* ctx, const ohip_node* nd, int i, int placement) {
  if (placement != OHIP_PLACE_DEVICE) return false;   // host results are the NCHW lanes
  auto nhwc = [&](int k) {
    return k < nd->n_inputs && nd->inputs[k].device && ohip_dtensor_layout(nd->inputs[k].device) == OHIP_NHWC;
  };
  const std::string op(nd->op_type);
  if (op == "QLinearConv") return i == 0 && attr_i(nd, "group", 1) == 1;
  if (op == "Conv") return i == 0 && conv_takes_nhwc(ctx, nd);
  if (op == "OhipConvInstanceNorm") {
    if (i == 0) return conv_takes_nhwc(ctx, nd);
    if (i != 5 || !nhwc(5)) return false;
    // the residual is read in place when it has the output's shape (whole 16-byte pixels)
    const ohip_tensor *x = input(nd, 0), *w = input(nd, 1), &r = nd->inputs[5];
    Geo g;
    std::string why;
    if (!x || !w || r.rank != 4 || !conv_geometry(nd, x, w, &g, &why)) return false;
    return r.shape[0] == g.n && r.shape[1] == g.cout && r.shape[2] == g.oh && r.shape[3] == g.ow &&
           ohip_dtensor_pitch_internal(r.device) == g.cout && g.cout % (16 / ebytes(r.dtype)) == 0;
  }
  if (op == "Slice" || op == "MaxPool") return i == 0;
  if (op == "Resize") {
    // NHWC in, NHWC out, when the session asks for an NHWC output (whole
    // 16-byte pixels, C per pixel)
    if (i != 0 || !nhwc(0) || attr_i(nd, "out_nhwc", 0) == 0) return false;
    const ohip_tensor& x = nd->inputs[0];
    return x.rank == 4 && ohip_dtensor_pitch_internal(x.device) == x.shape[1] &&
           (x.shape[1] * ebytes(x.dtype)) % 16 == 0;
  }
  if (op == "QLinearAdd") {
    if ((i != 0 && i != 3) || !nhwc(0) || !nhwc(3)) return false;
    const ohip_tensor &a = nd->inputs[0], &b = nd->inputs[3];
    if (a.rank != 4 || b.rank != 4) return false;
    for (int d = 0; d < 4; ++d) if (a.shape[d] != b.shape[d]) return false;
    return true;
  }
  if (op == "Concat") {
    if (nd->n_inputs < 1 || nd->inputs[0].rank != 4) return false;
    int64_t axis = attr_i(nd, "axis", 0);
    if (axis < 0) axis += 4;
    if (axis != 1) return false;
    for (int k = 0; k < nd->n_inputs; ++k) if (!nhwc(k)) return false;
    return true;
  }
  return false;
}

}  // namespace

// Resident NHWC operands that the node does not read in place are converted
// to NCHW first (into pool buffers released after the node is enqueued); the
// node then sees the layout of the reference's tensors.
extern "C" int ohip_try_dispatch(ohip_ctx* ctx, const ohip_node* node, int placement, ohip_output* out) {
  if (!ctx || !node || !node->op_type || !out) return OHIP_E_INVALID;
  std::memset(out, 0, sizeof(*out));
  for (int i = 0; i < node->n_inputs; ++i) {
    const ohip_tensor& t = node->inputs[i];
    if (t.device && !ohip_accepts_resident_slot(node->op_type, i)) {
      decline(std::string(node->op_type) + ": resident operand in host-read slot " + std::to_string(i));
      ohip_note_declined(ctx, t_err.c_str());
      return OHIP_DECLINED;
    }
  }
  std::vector<ohip_tensor> ins;
  std::vector<ohip_dtensor*> temps;
  for (int i = 0; i < node->n_inputs; ++i) {
    const ohip_tensor& t = node->inputs[i];
    if (!t.device || ohip_dtensor_layout(t.device) != OHIP_NHWC || takes_nhwc(ctx, node, i, placement)) continue;
    if (ins.empty()) ins.assign(node->inputs, node->inputs + node->n_inputs);
    const int64_t n = numel(&t);
    void* p = nullptr;
    int rc = ohip_malloc(ctx, (size_t)std::max<int64_t>(n * ebytes(t.dtype), 16), &p);
    if (rc == OHIP_OK) rc = ohip_dtensor_to_nchw_internal(ctx, t.device, p);
    ohip_dtensor* c = nullptr;
    if (rc == OHIP_OK) rc = ohip_dtensor_wrap(ctx, p, t.dtype, t.rank, t.shape, &c);
    if (rc) {
      if (p && !c) ohip_free(ctx, p);
      for (auto* x : temps) ohip_dtensor_free(x);
      return rc;
    }
    temps.push_back(c);
    ins[(size_t)i].device = c;
  }
  ohip_node local = *node;
  if (!ins.empty()) local.inputs = ins.data();
  const int rc = dispatch_node(ctx, &local, placement, out);
  for (auto* x : temps) ohip_dtensor_free(x);
  return rc;
}

namespace {

int dispatch_node(ohip_ctx* ctx, const ohip_node* node, int placement, ohip_output* out) {
  const std::string op(node->op_type);
  int rc;
  if (op == "Conv") rc = do_conv(ctx, node, placement, out);
  else if (op == "ConvTranspose") rc = do_conv_transpose(ctx, node, placement, out);
  else if (op == "Gemm") rc = do_gemm(ctx, node, false, placement, out);
  else if (op == "MatMul") rc = do_gemm(ctx, node, true, placement, out);
  else if (op == "QLinearMatMul") rc = do_qmatmul(ctx, node, true, placement, out);
  else if (op == "MatMulInteger") rc = do_qmatmul(ctx, node, false, placement, out);
  else if (op == "QLinearConv") rc = do_qconv(ctx, node, true, placement, out);
  else if (op == "ConvInteger") rc = do_qconv(ctx, node, false, placement, out);
  else if (op == "Relu") rc = do_unary(ctx, node, ohip::UN_RELU, placement, out);
  else if (op == "LeakyRelu") rc = do_unary(ctx, node, ohip::UN_LEAKY_RELU, placement, out);
  else if (op == "Tanh") rc = do_unary(ctx, node, ohip::UN_TANH, placement, out);
  else if (op == "Sigmoid") rc = do_unary(ctx, node, ohip::UN_SIGMOID, placement, out);
  else if (op == "Silu") rc = do_unary(ctx, node, ohip::UN_SILU, placement, out);
  else if (op == "Identity") rc = do_unary(ctx, node, ohip::UN_IDENTITY, placement, out);
  else if (op == "Add") rc = do_binary(ctx, node, ohip::BIN_ADD, placement, out);
  else if (op == "Sub") rc = do_binary(ctx, node, ohip::BIN_SUB, placement, out);
  else if (op == "Mul") rc = do_binary(ctx, node, ohip::BIN_MUL, placement, out);
  else if (op == "Div") rc = do_binary(ctx, node, ohip::BIN_DIV, placement, out);
  else if (op == "OxiInstanceNorm") rc = do_instnorm(ctx, node, false, placement, out);
  else if (op == "OhipConvInstanceNorm") rc = do_conv(ctx, node, placement, out, true);
  else if (op == "InstanceNormalization") rc = do_instnorm(ctx, node, true, placement, out);
  else if (op == "Resize") rc = do_resize(ctx, node, placement, out);
  else if (op == "Pad") rc = do_pad(ctx, node, placement, out);
  else if (op == "MaxPool") rc = do_maxpool(ctx, node, placement, out);
  else if (op == "Concat") rc = do_concat(ctx, node, placement, out);
  else if (op == "Slice") rc = do_slice(ctx, node, placement, out);
  else if (op == "Reshape" || op == "Flatten" || op == "Squeeze" || op == "Unsqueeze")
    rc = do_alias(ctx, node, op, placement, out);
  else if (op == "QuantizeLinear") rc = do_quantize(ctx, node, placement, out);
  else if (op == "DequantizeLinear") rc = do_dequantize(ctx, node, placement, out);
  else if (op == "QLinearAdd") rc = do_qadd(ctx, node, placement, out);
  else rc = decline("unsupported op " + op);
  if (rc == OHIP_DECLINED) ohip_note_declined(ctx, t_err.c_str());
  return rc;
}

}  // namespace

extern "C" void ohip_output_free(ohip_output* o) {
  if (!o) return;
  std::free(o->data);
  o->data = nullptr;
  if (o->device) ohip_dtensor_free(o->device);
  o->device = nullptr;
}
