# One-command build and test.
#   make check     build, CPU tests, then (when a GPU is visible) the GPU tests and smoke()
#   make build     compile the gfx950 library and the torch operator in place
#   make test      CPU tests (oracle, golden vectors, boundary, plan extents)
#   make test-gpu  GPU tests (parity, bit-exact properties, stream-K, capture, Muon)
#   make bench     the benchmark line (one GPU)
PY ?= python3
PYTEST_GPU = -u -m pytest tests -x -q -m gpu --timeout 300 --timeout-method thread

.PHONY: check build test test-gpu smoke bench

check: build test
	@if $(PY) -c "import sys, torch; sys.exit(0 if torch.cuda.is_available() else 1)"; then \
		$(PY) $(PYTEST_GPU) && $(PY) -c "import __graft_entry__ as g; g.smoke()"; \
	else \
		echo "no GPU visible: GPU tests skipped"; \
	fi

build:
	$(PY) -c "import __graft_entry__ as g; g.build()"

test:
	$(PY) -m pytest tests -x -q -m "not gpu"

test-gpu:
	$(PY) $(PYTEST_GPU)

smoke:
	$(PY) -c "import __graft_entry__ as g; g.smoke()"

bench:
	$(PY) bench.py
