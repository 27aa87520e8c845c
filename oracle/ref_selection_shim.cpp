// Exposes the reference's own selector header (compiled from where it lies in the
// reference tree, -I<reference>/src) through a C ABI so tests can compare the
// oracle's restatement and libsffft's selector against it. Test infrastructure.
#include <vector>

#include "selection.h"

extern "C" int ref_select_candidate(const char** method, const char** io, const char** config, const double* ms,
                                    const double* rel_err, int n, double max_error, const char* io_request) {
  std::vector<Candidate> v;
  for (int i = 0; i < n; i++) v.push_back({method[i], io[i], config[i], ms[i], rel_err[i]});
  const Candidate* best = select_candidate(v, max_error, io_request);
  return best ? (int)(best - v.data()) : -1;
}

extern "C" double ref_relative_l2(double squared_error, double squared_reference) {
  return relative_l2(squared_error, squared_reference);
}
