// Dense session (reference include/welvet/dense_session.hpp:12-19): one
// layer mounted at a fixed batch; execute many times on host buffers x
// [batch][in], pre and post [batch][out].
#pragma once

#include <cstddef>
#include <cstdint>

#include "welvet/activate.hpp"
#include "welvet/dtype.hpp"
#include "welvet/export.hpp"
#include "welvet/status.hpp"

namespace welvet::dense {

struct Session;

WELVET_API Status session_mount(int32_t batch, int32_t in, int32_t out, Activation act, DType dt,
                                const float* W_init, const double* bias, size_t bias_len,
                                Session** sess);

WELVET_API Status session_execute(Session* s, const float* x, float* pre, float* post);

WELVET_API void session_release(Session* s);

}  // namespace welvet::dense
