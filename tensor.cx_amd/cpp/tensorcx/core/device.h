// Device identity (interface of the reference's core/device.h:7-10).
#pragma once

#include <string>

namespace tensorcx {

struct Device {
  std::string type;
  int index{0};
};

}  // namespace tensorcx
