// Opaque session types of the C ABI (welvet_c.h), shared by the translation
// units that implement its entry points.
#pragma once

#include "welvet_c.h"

#include "layers.h"
#include "runtime.h"

// Dense session: one layer mounted at a fixed batch, its stream, workspace
// and the device buffers of the host-buffer execute.
struct welvet_dense_session {
  wv::Stream stream;
  wv::DenseLayer layer;
  wv::Workspace ws;
  int batch = 0;
  wv::DevBuf x, pre, post;
};
