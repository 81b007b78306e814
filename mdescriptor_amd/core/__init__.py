"""The public descriptor contract: batches, options, results, errors, control."""
