// Symbol visibility of the C++ layer/weights API. libwelvet.so is built with
// hidden visibility; the declarations in include/welvet/ that a caller links
// against carry WELVET_API.
#pragma once

#define WELVET_API __attribute__((visibility("default")))
