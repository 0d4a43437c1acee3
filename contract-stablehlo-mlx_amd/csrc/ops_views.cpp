// Views: reshape, transpose, broadcast and slice share the operand's buffer
// (mlx's reshape/transpose_axes/broadcast_to/slice, c/smlx_shim.c:203-229).
#include "ops.h"

namespace shlo {

static std::shared_ptr<Array> view_of(const ArrayP &a) {
  auto v = std::make_shared<Array>();
  v->buf = a->buf;
  v->offset = a->offset;
  v->dtype = a->dtype;
  v->shape = a->shape;
  v->strides = a->strides;
  return v;
}

ArrayP empty_array() { return new_array(kF32, Shape{0}); }

// Strides for viewing an array of shape `os` / strides `ost` as `ns` without
// moving data, when they exist: old and new dims are matched in groups of
// equal element count (outer to inner, size-1 old dims dropped); each group's
// old dims must nest (stride[i] == stride[i+1] * shape[i+1]), and its new
// dims then take strides from the group's innermost one (numpy's no-copy
// reshape rule).  A slice's rows split into heads, for one, stay a view.
static bool reshape_strides(const Shape &os, const Shape &ost, const Shape &ns, Shape *nst) {
  Shape od, ostr;
  for (size_t i = 0; i < os.size(); i++)
    if (os[i] != 1) od.push_back(os[i]), ostr.push_back(ost[i]);
  nst->assign(ns.size(), 0);
  size_t oi = 0, ni = 0;
  while (oi < od.size() && ni < ns.size()) {
    int64_t np = ns[ni], op = od[oi];
    size_t nj = ni + 1, oj = oi + 1;
    while (np != op) {
      if (np < op) {
        if (nj == ns.size()) return false;
        np *= ns[nj++];
      } else {
        if (oj == od.size()) return false;
        op *= od[oj++];
      }
    }
    for (size_t k = oi; k + 1 < oj; k++)
      if (ostr[k] != ostr[k + 1] * od[k + 1]) return false;
    (*nst)[nj - 1] = ostr[oj - 1];
    for (size_t k = nj - 1; k > ni; k--) (*nst)[k - 1] = (*nst)[k] * ns[k];
    oi = oj;
    ni = nj;
  }
  if (oi != od.size()) return false;
  for (; ni < ns.size(); ni++)
    if (ns[ni] != 1) return false;
  return true;
}

ArrayP reshape(const ArrayP &a, const Shape &shape) {
  if ((int)shape.size() > kMaxRank) fail("reshape: rank above 16");
  if (shape_count(shape) != a->size())
    fail(strf("reshape: %s has %lld elements, %s asks for %lld", shape_str(a->shape).c_str(),
              (long long)a->size(), shape_str(shape).c_str(), (long long)shape_count(shape)));
  Shape st;
  if (!a->contiguous() && a->size() > 0 && reshape_strides(a->shape, a->strides, shape, &st)) {
    auto v = view_of(a);
    v->shape = shape;
    v->strides = st;
    return v;
  }
  ArrayP src = a->contiguous() ? a : contiguous(a);
  auto v = view_of(src);
  v->shape = shape;
  v->strides = contiguous_strides(shape);
  v->shadow = src->shadow;
  return v;
}

ArrayP transpose(const ArrayP &a, const std::vector<int64_t> &perm) {
  const int r = a->rank();
  if ((int)perm.size() != r) fail(strf("transpose: %d axes for a rank-%d array", (int)perm.size(), r));
  std::vector<bool> seen(r, false);
  auto v = view_of(a);
  for (int i = 0; i < r; i++) {
    const int64_t p = perm[i];
    if (p < 0 || p >= r || seen[p]) fail("transpose: the axes are not a permutation");
    seen[p] = true;
    v->shape[i] = a->shape[p];
    v->strides[i] = a->strides[p];
  }
  return v;
}

Shape broadcast_shapes(const Shape &a, const Shape &b) {
  const size_t r = std::max(a.size(), b.size());
  Shape o(r);
  for (size_t i = 0; i < r; i++) {
    const int64_t da = i < r - a.size() ? 1 : a[i - (r - a.size())];
    const int64_t db = i < r - b.size() ? 1 : b[i - (r - b.size())];
    if (da != db && da != 1 && db != 1)
      fail("broadcast: shapes " + shape_str(a) + " and " + shape_str(b) + " do not broadcast");
    o[i] = da == 1 ? db : da;
  }
  return o;
}

ArrayP broadcast_to(const ArrayP &a, const Shape &shape) {
  if ((int)shape.size() > kMaxRank) fail("broadcast: rank above 16");
  if (shape.size() < a->shape.size())
    fail("broadcast: cannot broadcast " + shape_str(a->shape) + " to " + shape_str(shape));
  auto v = view_of(a);
  const size_t lead = shape.size() - a->shape.size();
  v->shape = shape;
  v->strides.assign(shape.size(), 0);
  for (size_t i = 0; i < a->shape.size(); i++) {
    const int64_t d = a->shape[i], o = shape[lead + i];
    if (d == o) v->strides[lead + i] = a->strides[i];
    else if (d == 1) v->strides[lead + i] = 0;
    else fail("broadcast: cannot broadcast " + shape_str(a->shape) + " to " + shape_str(shape));
  }
  if (a->size() == shape_count(shape)) v->shadow = a->shadow;
  return v;
}

ArrayP slice(const ArrayP &a, const Shape &start, const Shape &stop, const Shape &step) {
  const int r = a->rank();
  if ((int)start.size() != r || (int)stop.size() != r || (int)step.size() != r)
    fail(strf("slice: %d/%d/%d indices for a rank-%d array", (int)start.size(), (int)stop.size(),
              (int)step.size(), r));
  auto v = view_of(a);
  for (int i = 0; i < r; i++) {
    const int64_t d = a->shape[i];
    if (step[i] <= 0) fail("slice: strides must be positive");
    const int64_t s = std::min(std::max<int64_t>(start[i], 0), d);
    const int64_t e = std::min(std::max<int64_t>(stop[i], s), d);
    const int64_t n = (e - s + step[i] - 1) / step[i];
    v->offset += s * a->strides[i];
    v->shape[i] = n;
    v->strides[i] = a->strides[i] * step[i];
  }
  if (v->size() == 0) v->buf = nullptr, v->offset = 0;
  return v;
}

}  // namespace shlo
