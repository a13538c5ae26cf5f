"""TileMix attention: routing maps, the dense-batch entry and the HIP launch layer."""
