// pp_inst_maxmin_f64.hip -- instantiation of the numeric drivers for MaxMin<double>.
#include "pp_kernels.h"

namespace pp {
template std::string factor_impl<MaxMin<double>>(pp_ctx *, pp_fac *, const void *);
template std::string packs_impl<MaxMin<double>>(pp_ctx *, pp_fac *);
template std::string star_impl<MaxMin<double>>(pp_ctx *, const pp_fac *, void *, i64, int);
template std::string star_src_impl<MaxMin<double>>(pp_ctx *, const pp_fac *, const RowSub &, i64, int, void *, i64);
template std::string solve_impl<MaxMin<double>>(pp_ctx *, const pp_fac *, void *, i64, i64, bool, bool, void *);
template std::string gemm_impl<MaxMin<double>>(pp_ctx *, i64, i64, i64, const void *, i64, const void *, i64, void *, i64);
template std::string getrf_impl<MaxMin<double>>(pp_ctx *, i64, i64, void *, void *, void *);
}  // namespace pp
