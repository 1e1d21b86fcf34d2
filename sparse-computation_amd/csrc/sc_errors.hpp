// sc_errors.hpp -- status codes and the thread-local last-error text behind
// the C ABI.  C++ exceptions (sc::Error, std::bad_alloc, anything else) are
// caught at the boundary and turned into a status code plus a message.
#pragma once

#include <new>
#include <string>

#include "sc_api.h"

namespace sc {

void set_last_error(const std::string &msg);
void clear_last_error();

}  // namespace sc

// Run the lambda (returning void) and translate exceptions to codes.
#define SC_GUARD(...)                                           \
  do {                                                          \
    try {                                                       \
      sc::clear_last_error();                                   \
      (__VA_ARGS__)();                                          \
      return SC_OK;                                             \
    } catch (const sc::Error &e_) {                             \
      sc::set_last_error(e_.msg);                               \
      return e_.code;                                           \
    } catch (const std::bad_alloc &) {                          \
      sc::set_last_error("out of host memory");                 \
      return SC_ERR_NOMEM;                                      \
    } catch (const std::exception &e_) {                        \
      sc::set_last_error(e_.what());                            \
      return SC_ERR_INTERNAL;                                   \
    } catch (...) {                                             \
      sc::set_last_error("unknown C++ exception");              \
      return SC_ERR_INTERNAL;                                   \
    }                                                           \
  } while (0)
