// SPDX-License-Identifier: Apache-2.0
// ref_distance_wrap.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Exports the reference's own CPU distance primitives (the header-only
// src/Distance.h:26-81 of the reference tree, included from where it lies, not
// copied) as C symbols, so tests can check the oracle's restatement against the
// reference code bit for bit. Built by `make ref` in this directory into
// oracle/_ref/ only when the reference tree is present. The rest of the
// reference's flat path (src/FlatIndex.mm) needs Apple Foundation/Metal and
// cannot be compiled on Linux.
#include "Distance.h"

extern "C" {
float ref_dot(const float* a, const float* b, int dim) { return mflat::detail::dot(a, b, dim); }
float ref_sql2(const float* a, const float* b, int dim) { return mflat::detail::sqL2(a, b, dim); }
void ref_row_sq_norms(const float* v, int n, int dim, float* out) {
    mflat::detail::rowSqNorms(v, n, dim, out);
}
void ref_normalize_rows(float* v, int n, int dim) { mflat::detail::normalizeRows(v, n, dim); }
float ref_score(int metric, const float* q, const float* d, int dim) {
    return mflat::detail::score(static_cast<mflat::Metric>(metric), q, d, dim);
}
float ref_score_to_value(int metric, float s) {
    return mflat::detail::scoreToValue(static_cast<mflat::Metric>(metric), s);
}
float ref_empty_value(int metric) {
    return mflat::detail::emptyValue(static_cast<mflat::Metric>(metric));
}
float ref_l2_score_from_dot(float qn, float dn, float dotqd) {
    return mflat::detail::l2ScoreFromDot(qn, dn, dotqd);
}
}
