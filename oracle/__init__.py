"""CPU oracle (test infrastructure only): see tsne_oracle.cpp."""
